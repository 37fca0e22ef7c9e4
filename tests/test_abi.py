"""CPU checks of the C-ABI library: it loads, exports every declared symbol, and its
host-side queries and argument rejections work without touching a GPU."""

import ctypes as ct
import json
import re
from pathlib import Path

import pytest

from ascendflow_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "ascendflow_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    return _native.library()


def test_header_declares_exactly_the_bound_symbols():
    assert declared_functions() == sorted(_native.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_kernel_config_and_workspace_queries(lib):
    for kernel, tensors in (("sparse_mla", 13), ("attention_target", 4), ("simple_attention", 4)):
        cfg = (ct.c_int64 * 5)()
        assert getattr(lib, f"kernel_config_{kernel}")(cfg) == 0
        has_workspace = kernel == "sparse_mla"
        assert cfg[0] == tensors and cfg[2] == int(has_workspace) and cfg[3] == 256 and cfg[4] == 4
        meta = json.loads(getattr(lib, f"kernel_metadata_{kernel}")().decode())
        # The reference's schema (src/backend/abi.py:19-59, consumed by
        # src/runtime/torch.py:94-167): name, target, tensors with dtype,
        # shape, layout and access, parameters with minimum and multiple.
        assert meta["version"] == 1 and meta["name"] == kernel and meta["target"] == "gfx950"
        assert len(meta["tensors"]) == tensors
        for spec in meta["tensors"]:
            assert set(spec) == {"name", "dtype", "shape", "layout", "access"}
            assert spec["layout"] == "linear" and spec["access"] in ("read", "write")
            assert all(isinstance(n, (int, str)) for n in spec["shape"])
            assert spec["dtype"] in ("bf16", "f16", "f32", "i32") or spec["dtype"] in meta.get("dtypes", {})
        for spec in meta["parameters"]:
            assert set(spec) == {"name", "minimum", "multiple"} and spec["minimum"] >= 1 and spec["multiple"] >= 1
            assert any(spec["name"] in t["shape"] for t in meta["tensors"])
        assert meta["disjoint_external"] is True and meta["workspace"] is has_workspace
    size = ct.c_uint64(123)
    # The sparse workspace is the row-list plan: T counts rounded up to 256
    # bytes, then T lists of WINDOW + TOPK entries rounded up to 256.
    params = good_params(parts=1)
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 256 + 16 * 768 * 4
    params = good_params(T=100, TOPK=1000, S=1128, parts=1)
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 512 + 100 * 1280 * 4
    # Split keys add partial records: (split keys) * P * (2 * BM * D + BM * BM / 2)
    # bytes (normalised b16 outputs plus FP32 max and denominator). Only streams
    # of at most one full round of 256 keys split, the keys beyond the full
    # round into the P (r P <= 256) that the library's cost model finds
    # cheapest, if any beats the whole round: T = 16 into 7 parts (3 chunks
    # each), T = 100 with 36 chunks into 2; not decode T = 384 (128 keys beyond
    # the round: HBM-bound parts plus the merge cost more than 20 latency-bound
    # steps) or T = 512 (two full rounds).
    per_part = 2 * 64 * 512 + 64 * 64 // 2
    params = good_params()
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 49408 + 16 * 7 * per_part
    params = good_params(T=100, TOPK=1000, S=1128)
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 512512 + 100 * 2 * per_part
    params = good_params(T=384)
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 1536 + 384 * 768 * 4
    params = good_params(T=512)
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 2048 + 512 * 768 * 4
    params = good_params(T=512, parts=3)  # forced: every key in 3 parts
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(params)) == 0
    assert size.value == 2048 + 512 * 768 * 4 + 512 * 3 * per_part
    for parts in (-1, 9):
        assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(good_params(parts=parts))) == -2
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(good_params(WINDOW=0, TOPK=0, S=0))) == -2
    assert lib.workspace_size_sparse_mla(ct.byref(size), None) == -1
    assert lib.workspace_size_sparse_mla(None, None) == -1
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(good_params(D=64))) == -2
    assert lib.workspace_size_attention_target(ct.byref(size), 8, 8, None) == 0 and size.value == 0
    assert lib.workspace_size_simple_attention(None, 64, 1) == -1
    assert b"gfx950" in lib.ascendflow_amd_version()


def test_sparse_metadata_lists_tensors_in_reference_order(lib):
    from oracle.sparse_reference import TENSOR_ORDER

    meta = json.loads(lib.kernel_metadata_sparse_mla().decode())
    assert tuple(t["name"] for t in meta["tensors"]) == TENSOR_ORDER
    assert [t["access"] for t in meta["tensors"]].count("write") == 1


def good_params(**overrides):
    fields = dict(B=4, T=16, H=64, D=512, PAGE=128, RATIO=2, MAX_SEQ=4096, ORI_BLOCKS=128, CMP_BLOCKS=128,
                  WINDOW=128, TOPK=512, S=640, BM=64, dtype=0, scale=0.044, parts=0, debug_rows=None)
    fields.update(overrides)
    return _native.SparseMlaParams(**fields)


@pytest.mark.parametrize(
    "overrides,status",
    [
        ({"D": 384}, -2),
        ({"BM": 16}, -2),
        ({"H": 96}, -2),
        ({"RATIO": 3}, -2),
        ({"S": 100}, -2),
        ({"scale": 0.0}, -2),
        ({"ring": 2}, -2),
        ({"ring": 5}, -2),
        ({"dtype": 7}, -3),
        ({"ORI_BLOCKS": 1 << 24}, -2),
        # No gather slot at all: nothing to stream (the row lists would be empty).
        ({"WINDOW": 0, "TOPK": 0, "S": 0}, -2),
    ],
)
def test_sparse_launcher_rejects_bad_configurations_before_any_launch(lib, overrides, status):
    params = good_params(**overrides)
    args = [None] + [ct.c_void_p(16)] * 13 + [None]
    assert lib.launch_sparse_mla(*args, ct.byref(params)) == status


def test_launchers_reject_null_arguments(lib):
    params = good_params()
    assert lib.launch_sparse_mla(*([None] * 15), None) == -1
    assert lib.launch_sparse_mla(*([None] * 15), ct.byref(params)) == -1
    assert lib.launch_sparse_mla_gather(*([None] * 13), ct.byref(params)) == -1
    assert lib.launch_sparse_mla_planned(*([None] * 7), ct.byref(params)) == -1
    assert lib.launch_sparse_mla_planned(*([None] * 7), None) == -1
    p = ct.c_void_p(16)
    debug = good_params(debug_rows=16)
    assert lib.launch_sparse_mla_planned(None, p, p, p, p, p, p, ct.byref(debug)) == -2
    assert lib.launch_sparse_mla_planned(None, p, p, p, p, p, p, ct.byref(good_params(ring=5))) == -2
    fa = _native.FaParams(B=1, HQ=8, HKV=8, D=128, dtype=1, causal=0, scale=0.088, reserved=0)
    assert lib.launch_attention_target(None, None, None, None, None, None, 8, 8, ct.byref(fa)) == -1
    p = ct.c_void_p(16)
    assert lib.launch_attention_target(None, p, p, p, p, None, 0, 8, ct.byref(fa)) == -2
    fa.HKV = 3
    assert lib.launch_attention_target(None, p, p, p, p, None, 8, 8, ct.byref(fa)) == -2
    assert lib.launch_simple_attention(None, p, p, p, p, None, 100, 1) == -2
    assert lib.launch_cache_flush(None, None, 1024) == -1
    assert lib.launch_clock_probe(None, None, 1000) == -1
    assert lib.launch_clock_probe(None, ct.c_void_p(16), 0) == -2


@pytest.mark.parametrize(
    "fields,status",
    [
        (dict(B=2, T=8, TOPK=512, RATIO=2, C=4096), -1),  # NULL tensors
        (dict(B=0, T=8, TOPK=512, RATIO=2, C=4096), -2),
        (dict(B=2, T=8, TOPK=0, RATIO=2, C=4096), -2),
        (dict(B=2, T=8, TOPK=512, RATIO=3, C=4096), -2),
        (dict(B=2, T=8, TOPK=512, RATIO=2, C=0), -2),
        (dict(B=2, T=8, TOPK=512, RATIO=2, C=2**31), -2),
    ],
)
def test_topk_launcher_rejects_bad_arguments_before_any_launch(lib, fields, status):
    from ascendflow_amd.sparse_attention.indexer import SparseTopkParams

    params = SparseTopkParams(**fields)
    assert lib.launch_sparse_topk_indices(None, None, None, None, None, None, ct.byref(params)) == status
    assert lib.launch_sparse_topk_indices(None, None, None, None, None, None, None) == -1


def test_python_entries_check_the_reference_asserts_before_launching():
    from ascendflow_amd.sparse_attention.attention import check_policy

    good = dict(B=4, T=16, H=64, D=512, PAGE=128, RATIO=2, MAX_SEQ=4096, WINDOW=128, TOPK=512, ROWS=32, S=640,
                BM=64, PARTS=1, GROUPS=20, VR=16, BK=512, C=128, SCALE=0.044)
    check_policy(**good)
    for bad in ({"WINDOW": 64}, {"S": 512}, {"BM": 48}, {"VR": 3}, {"RATIO": 4}, {"SCALE": -1.0}, {"PARTS": 2}):
        with pytest.raises(ValueError):
            check_policy(**dict(good, **bad))
    from ascendflow_amd.flash_attention import causal_policy

    assert causal_policy(1000, 9000) == {"kv_tile": 256, "vector_rows": 16}
    assert causal_policy(4096, 4096) == {"kv_tile": 512, "vector_rows": 16}
    assert causal_policy(8192, 8192) == {"kv_tile": 1024, "vector_rows": 8}


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _native.library(tmp_path / "absent.so")


def test_framework_op_is_registered_with_a_shape_only_fake():
    """ascendflow_amd::sparse_flash_mla traces on meta tensors (no GPU, no
    launch): output [T, H, D] in the query dtype, softmax_lse f32 [T, H] or empty."""
    import torch

    import ascendflow_amd.sparse_attention  # noqa: F401  registers the op

    meta = torch.device("meta")
    t, h, d = 6, 64, 512
    i32 = lambda *shape: torch.empty(*shape, dtype=torch.int32, device=meta)  # noqa: E731
    args = (torch.empty(t, h, d, dtype=torch.bfloat16, device=meta),
            torch.empty(32, 128, 1, d, dtype=torch.bfloat16, device=meta),
            torch.empty(32, 64, 1, d, dtype=torch.bfloat16, device=meta),
            i32(t, 1, 512), i32(2, 16), i32(2, 16), i32(3), i32(2), i32(2), i32(2), i32(t, 1),
            torch.empty(h, device=meta), 512 ** -0.5, 2)
    out, lse = torch.ops.ascendflow_amd.sparse_flash_mla(*args, return_softmax_lse=True)
    assert out.shape == (t, h, d) and out.dtype == torch.bfloat16
    assert lse.shape == (t, h) and lse.dtype == torch.float32
    _, empty = torch.ops.ascendflow_amd.sparse_flash_mla(*args)
    assert empty.numel() == 0


def test_topk_op_is_registered_with_a_shape_only_fake():
    """ascendflow_amd::sparse_topk_indices traces on meta tensors: [T, 1, topk] int32."""
    import torch

    import ascendflow_amd.sparse_attention  # noqa: F401  registers the op

    meta = torch.device("meta")
    i32 = lambda *shape: torch.empty(*shape, dtype=torch.int32, device=meta)  # noqa: E731
    out = torch.ops.ascendflow_amd.sparse_topk_indices(torch.empty(6, 4096, device=meta), i32(3), i32(2), i32(2), 512, 2)
    assert out.shape == (6, 1, 512) and out.dtype == torch.int32


def test_noalloc_entry_rejects_workspaces_beyond_its_scratch(lib):
    """A call whose workspace exceeds the 32 MiB static scratch is refused with
    AFA_E_WORKSPACE before anything is launched (a 32K-token prefill needs 100 MiB)."""
    big = good_params(B=1, T=32768, MAX_SEQ=32768, parts=1)
    size = ct.c_uint64(0)
    assert lib.workspace_size_sparse_mla(ct.byref(size), ct.byref(big)) == 0 and size.value > _native.SCRATCH_BYTES
    args = [None] + [ct.c_void_p(16)] * 13
    assert lib.launch_sparse_mla_noalloc(*args, ct.byref(big)) == -4
    assert lib.launch_sparse_mla_noalloc(*args, ct.byref(good_params(D=64))) == -2
    assert lib.launch_sparse_mla_noalloc(*args, None) == -1


def test_disjointness_check_covers_written_tensors_only():
    """A written tensor may overlap nothing; read tensors may share memory
    (src/runtime/torch.py:94-167 checks the same disjointness)."""
    import torch

    from ascendflow_amd._tensors import check_disjoint

    buf = torch.zeros(64)
    a, b, c = buf[0:16], buf[8:24], buf[32:48]
    check_disjoint([("a", a, False), ("b", b, False), ("c", c, True)])  # reads overlap: allowed
    with pytest.raises(ValueError, match="a and b overlap"):
        check_disjoint([("a", a, False), ("b", b, True), ("c", c, False)])
    with pytest.raises(ValueError, match="a and c overlap"):
        check_disjoint([("a", buf[0:40], False), ("b", b, False), ("c", c, True)])
    check_disjoint([("a", a, True), ("e", buf[0:0], False)])  # empty tensors never overlap
