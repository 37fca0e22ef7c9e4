"""ctypes binding of the C-ABI library ``libascendflow_amd.so`` (include/ascendflow_amd.h).

The library is built in-tree by ``ascendflow_amd.build.build()``. There is no
fallback: if the library is missing or a symbol is absent, loading raises, so a
product call can never silently run anything but the HIP kernels.
"""

from __future__ import annotations

import ctypes as ct
from pathlib import Path

LIB_NAME = "libascendflow_amd.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

AFA_DTYPE = {"bf16": 0, "f16": 1}
SCRATCH_BYTES = 32 << 20  # AFA_SCRATCH_BYTES: the allocation-free entry's static workspace per GPU
STATUS = {
    -1: "AFA_E_NULL: a required pointer is NULL",
    -2: "AFA_E_SHAPE: unsupported or inconsistent size",
    -3: "AFA_E_DTYPE: unsupported storage dtype",
    -4: "AFA_E_WORKSPACE: workspace missing or too small",
}

# Every symbol include/ascendflow_amd.h declares.
EXPORTS = (
    "launch_sparse_mla",
    "launch_sparse_mla_noalloc",
    "launch_sparse_mla_gather",
    "launch_sparse_mla_plan",
    "launch_sparse_mla_planned",
    "launch_gather_probe",
    "launch_sparse_topk_indices",
    "launch_attention_target",
    "launch_simple_attention",
    "kernel_config_sparse_mla",
    "kernel_config_attention_target",
    "kernel_config_simple_attention",
    "kernel_metadata_sparse_mla",
    "kernel_metadata_attention_target",
    "kernel_metadata_simple_attention",
    "workspace_size_sparse_mla",
    "workspace_size_attention_target",
    "workspace_size_simple_attention",
    "launch_cache_flush",
    "launch_clock_probe",
    "ascendflow_amd_version",
)


class SparseMlaParams(ct.Structure):
    _fields_ = [
        ("B", ct.c_int32),
        ("T", ct.c_int32),
        ("H", ct.c_int32),
        ("D", ct.c_int32),
        ("PAGE", ct.c_int32),
        ("RATIO", ct.c_int32),
        ("MAX_SEQ", ct.c_int32),
        ("ORI_BLOCKS", ct.c_int32),
        ("CMP_BLOCKS", ct.c_int32),
        ("WINDOW", ct.c_int32),
        ("TOPK", ct.c_int32),
        ("S", ct.c_int32),
        ("BM", ct.c_int32),
        ("dtype", ct.c_int32),
        ("scale", ct.c_float),
        ("parts", ct.c_int32),
        ("ring", ct.c_int32),
        ("debug_rows", ct.c_void_p),
        ("softmax_lse", ct.c_void_p),
    ]


class FaParams(ct.Structure):
    _fields_ = [
        ("B", ct.c_int32),
        ("HQ", ct.c_int32),
        ("HKV", ct.c_int32),
        ("D", ct.c_int32),
        ("dtype", ct.c_int32),
        ("causal", ct.c_int32),
        ("scale", ct.c_float),
        ("reserved", ct.c_int32),
    ]


_P = ct.c_void_p
_SIGNATURES = {
    "launch_sparse_mla": ([_P] * 15 + [ct.POINTER(SparseMlaParams)], ct.c_int),
    "launch_sparse_mla_noalloc": ([_P] * 14 + [ct.POINTER(SparseMlaParams)], ct.c_int),
    "launch_sparse_mla_gather": ([_P] * 13 + [ct.POINTER(SparseMlaParams)], ct.c_int),
    "launch_sparse_mla_plan": ([_P] * 10 + [ct.POINTER(SparseMlaParams)], ct.c_int),
    "launch_sparse_mla_planned": ([_P] * 7 + [ct.POINTER(SparseMlaParams)], ct.c_int),
    "launch_gather_probe": (
        [_P] * 4 + [ct.POINTER(SparseMlaParams), ct.c_int32, ct.c_int32, ct.c_int32, _P],
        ct.c_int,
    ),
    "launch_sparse_topk_indices": ([_P] * 7, ct.c_int),
    "launch_attention_target": (
        [_P] * 6 + [ct.c_int64, ct.c_int64, ct.POINTER(FaParams)],
        ct.c_int,
    ),
    "launch_simple_attention": ([_P] * 6 + [ct.c_int64, ct.c_int64], ct.c_int),
    "kernel_config_sparse_mla": ([ct.POINTER(ct.c_int64)], ct.c_int),
    "kernel_config_attention_target": ([ct.POINTER(ct.c_int64)], ct.c_int),
    "kernel_config_simple_attention": ([ct.POINTER(ct.c_int64)], ct.c_int),
    "kernel_metadata_sparse_mla": ([], ct.c_char_p),
    "kernel_metadata_attention_target": ([], ct.c_char_p),
    "kernel_metadata_simple_attention": ([], ct.c_char_p),
    "workspace_size_sparse_mla": ([ct.POINTER(ct.c_uint64), ct.POINTER(SparseMlaParams)], ct.c_int),
    "workspace_size_attention_target": (
        [ct.POINTER(ct.c_uint64), ct.c_int64, ct.c_int64, ct.POINTER(FaParams)],
        ct.c_int,
    ),
    "workspace_size_simple_attention": (
        [ct.POINTER(ct.c_uint64), ct.c_int64, ct.c_int64],
        ct.c_int,
    ),
    "launch_cache_flush": ([_P, _P, ct.c_uint64], ct.c_int),
    "launch_clock_probe": ([_P, _P, ct.c_int32], ct.c_int),
    "ascendflow_amd_version": ([], ct.c_char_p),
}

_lib = None


def library(path: Path | None = None) -> ct.CDLL:
    """Load (once) and return the C-ABI library; raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = Path(path) if path is not None else LIB_PATH
    if not target.exists():
        raise RuntimeError(
            f"{target} is missing: build the HIP extension first "
            "(python -c 'import __graft_entry__ as g; g.build()'). There is no CPU fallback."
        )
    lib = ct.CDLL(str(target))
    for name, (argtypes, restype) in _SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError names a missing export
        fn.argtypes = argtypes
        fn.restype = restype
    if path is None:
        _lib = lib
    return lib


def check(status: int, what: str) -> None:
    """Turn a launcher status into an exception (no retry, as the reference)."""
    if status == 0:
        return
    if status < 0:
        raise ValueError(f"{what} rejected: {STATUS.get(status, status)}")
    raise RuntimeError(f"{what} failed: hipError_t {status}")
