"""bench.py's command-line contract, on the CPU (no GPU work is reached).

The driver runs ``python bench.py --gpus N --steps K --warmup W``; this build
measures one GPU, so any other N must exit non-zero with a message saying so
(before touching the GPU), and the usual flags must parse.
"""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    for n in ("2", "8"):
        done = run_bench("--gpus", n, "--steps", "3", "--warmup", "1")
        assert done.returncode == 2, done.stderr
        assert "measures one GPU" in done.stderr
        assert done.stdout == ""  # no JSON line for an unmeasured configuration


def test_help_lists_the_driver_flags():
    done = run_bench("--help")
    assert done.returncode == 0, done.stderr
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in done.stdout
