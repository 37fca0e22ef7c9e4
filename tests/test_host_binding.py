"""CPU checks of sparse_mla's host side: the per-(device, stream, sizes) binding
cache that replaces per-call validation work (the reference's KernelLaunch per
(stream, sizes), src/runtime/torch.py:170-186), and the disjointness contract
that covers every written operand (output, workspace, softmax_lse, debug image)."""

import pytest
import torch

from ascendflow_amd._tensors import check_disjoint
from ascendflow_amd.sparse_attention import attention as A

POLICY = dict(B=4, T=16, H=64, D=512, PAGE=128, RATIO=2, MAX_SEQ=4096, ORI_BLOCKS=128, CMP_BLOCKS=128, WINDOW=128,
              TOPK=512, S=640, BM=64, SCALE=0.04419417382415922)
ORDER = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW", "TOPK", "S", "BM", "SCALE")


def sizes(dtype="bf16", parts=None, ring=None, **over):
    p = dict(POLICY, **over)
    return (p["B"], p["T"], p["H"], p["D"], p["PAGE"], p["RATIO"], p["MAX_SEQ"], p["ORI_BLOCKS"], p["CMP_BLOCKS"],
            p["WINDOW"], p["TOPK"], 32, p["S"], p["BM"], 1, 20, 16, 512, 128, dtype, p["SCALE"], parts, ring)


def make(stream=7, dtype="bf16", **over):
    p = dict(POLICY, **over)
    return A._binding(torch.device("cuda", 0), stream, sizes(dtype, **over), tuple(p[k] for k in ORDER), dtype, 0, 0)


@pytest.fixture(autouse=True)
def fresh_cache():
    A.release_bindings()
    yield
    A.release_bindings()


def test_binding_key_separates_sizes_dtype_and_stream():
    base = make()
    assert make() is base  # same device, stream and sizes: one binding
    others = [make(stream=8), make(dtype="f16"), make(T=32), make(TOPK=256, S=640), make(B=2),
              make(MAX_SEQ=8192), make(BM=32)]
    assert all(o is not base for o in others)
    assert len({id(o) for o in others}) == len(others)
    keys = {A.binding_key(0, 7, sizes()), A.binding_key(1, 7, sizes()), A.binding_key(0, 8, sizes()),
            A.binding_key(0, 7, sizes("f16")), A.binding_key(0, 7, sizes(parts=2)), A.binding_key(0, 7, sizes(ring=4))}
    assert len(keys) == 6


def test_binding_key_separates_libraries():
    """A binding (and its workspace, sized by the library's own workspace
    query) belongs to the library that made it: with another library loaded
    in its place the same call gets a new binding."""
    from ascendflow_amd import _native
    base = make()
    saved = _native._lib
    try:
        _native._lib = _native.library(_native.LIB_PATH)  # a second handle of the library
        assert A.binding_key(0, 7, sizes()) != (id(saved), 0, 7) + sizes()
        assert make() is not base
    finally:
        _native._lib = saved
    assert make() is base


def test_binding_holds_the_calls_parameters_and_workspace_size():
    b = make(T=1024)
    assert (b.params.T, b.params.B, b.params.TOPK, b.params.dtype) == (1024, 4, 512, 0)
    assert b.params.debug_rows is None and b.params.softmax_lse is None
    assert b.nbytes == A.workspace_bytes(**dict(POLICY, T=1024))
    assert tuple(b.specs[0][1]) == (1024, 64, 512) and b.specs[-1][0] == "attention_out"
    assert b.specs[0][2] is torch.bfloat16 and make(dtype="f16").specs[0][2] is torch.float16


def test_binding_cache_is_bounded():
    first = make(stream=1000)
    for k in range(A.MAX_BINDINGS):
        make(stream=k)
    assert len(A._bindings) == A.MAX_BINDINGS
    assert make(stream=1000) is not first  # evicted, rebuilt


def test_lse_carved_out_of_the_workspace_is_rejected():
    workspace = torch.empty(1 << 16, dtype=torch.uint8)
    lse = workspace[: 16 * 64 * 4].view(torch.float32).view(16, 64)
    q = torch.empty(16, 64, 512, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    with pytest.raises(ValueError, match="overlap"):
        check_disjoint([("q", q, False), ("attention_out", out, True), ("workspace", workspace, True),
                        ("softmax_lse", lse, True)])
    # the same operands with a separate LSE pass
    check_disjoint([("q", q, False), ("attention_out", out, True), ("workspace", workspace, True),
                    ("softmax_lse", torch.empty(16, 64), True)])


def test_debug_image_overlapping_the_output_is_rejected():
    out = torch.empty(16, 64, 512, dtype=torch.bfloat16)
    debug = out.view(torch.int32)[:1]  # a view into the output
    with pytest.raises(ValueError, match="overlap"):
        check_disjoint([("attention_out", out, True), ("debug_rows", debug, True)])
