"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

``tests/host/abi_host_checks.cpp`` calls every host-side path of the C ABI
that returns before a launch: argument validation and rejections, workspace
sizing (with the split cost model), metadata, config and version queries.
It is built here together with the library sources, the sanitizers on the
host compilation only (the device code is compiled as usual and never runs,
so no GPU is needed), and run on the CPU; any memory error or undefined
behaviour aborts it.
"""

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HOST_SANITIZERS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                   "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def test_host_abi_checks_under_sanitizers(tmp_path):
    from ascendflow_amd.build import HIP_FLAGS, hipcc

    compiler = hipcc()
    if not Path(compiler).exists():
        pytest.skip(f"{compiler} is not installed")
    flags = ["-O1" if f == "-O3" else f for f in HIP_FLAGS] + HOST_SANITIZERS
    sources = sorted((ROOT / "ascendflow_amd" / "csrc").glob("*.hip")) + [ROOT / "tests" / "host" / "abi_host_checks.cpp"]

    def compile_one(src):
        obj = tmp_path / (src.stem + ".o")
        lang = ["-x", "hip"] if src.suffix == ".cpp" else []
        done = subprocess.run([compiler, *flags, *lang, "-c", str(src), "-o", str(obj)], capture_output=True, text=True)
        assert done.returncode == 0, done.stderr[-4000:]
        return obj

    with ThreadPoolExecutor(4) as pool:
        objects = list(pool.map(compile_one, sources))
    exe = tmp_path / "abi_host_checks"
    link = subprocess.run([compiler, "--offload-arch=gfx950", *HOST_SANITIZERS, *map(str, objects), "-o", str(exe)],
                          capture_output=True, text=True)
    assert link.returncode == 0, link.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-6000:]
    assert "host ABI checks passed" in run.stdout
