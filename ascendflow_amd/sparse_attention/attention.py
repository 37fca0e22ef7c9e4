"""TND sparse shared-KV attention (DeepSeek V4.1 sparse MLA) on MI355X.

Drop-in for ``examples/sparse_attention/attention.py:210-246`` (``sparse_mla``):
same tensor arguments in the same order, same constexpr keywords and defaults.
The call launches the fused gfx950 kernel of ``csrc/sparse_mla.hip`` through
the C ABI ``launch_sparse_mla`` on the current PyTorch-ROCm stream and returns
without synchronising, as the reference launcher does
(``docs/guide/runtime.md:86-89``).

Tiling constexprs that only describe the Ascend pipeline (ROWS, GROUPS, VR, BK,
C, PARTS) are accepted and checked against the reference's own asserts
(``attention.py:253-262``) so that the same calls are valid or rejected, but
they do not change the gfx950 schedule.
"""

from __future__ import annotations

import ctypes as ct
import functools
from collections import OrderedDict

import torch

from .. import _native
from .._native import SparseMlaParams
from .._tensors import DTYPES, check_disjoint, check_tensor, require, storage_dtype, stream_handle


def check_policy(B, T, H, D, PAGE, RATIO, MAX_SEQ, WINDOW, TOPK, ROWS, S, BM, PARTS, GROUPS, VR, BK, C, SCALE):
    """The reference's specialisation asserts (``attention.py:253-262``)."""
    require(0 < B < 2**31 and 0 < T < 2**31, "nonempty INT32 TND prefix")
    require(H % BM == 0 and BM in (32, 64), "complete head tiles")
    require(WINDOW == 128 and PAGE == 128 and BK == 512 and C == 128, "cache/tile geometry")
    require(D % C == 0 and S == WINDOW + -(-TOPK // BK) * BK, "complete selected capacities")
    require(PARTS == 1 and ROWS in (16, 32) and GROUPS > 0, "sparse query policy")
    require(VR in (4, 8, 16) and (BM // 2) % VR == 0, "softmax row groups")
    require(RATIO in (1, 2) and MAX_SEQ % PAGE == 0, "complete C1/C2 pages")
    require(-(-S // 512) * 512 <= 4096, "resident softmax capacity")
    require(SCALE > 0.0, "positive attention scale")
    require(D in (128, 256, 512), "gfx950 kernel supports D in {128, 256, 512}")


def make_params(B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM, dtype, SCALE, debug_rows=None,
                parts=0, softmax_lse=None, ring=0):
    return _native.SparseMlaParams(
        B=B,
        T=T,
        H=H,
        D=D,
        PAGE=PAGE,
        RATIO=RATIO,
        MAX_SEQ=MAX_SEQ,
        ORI_BLOCKS=ORI_BLOCKS,
        CMP_BLOCKS=CMP_BLOCKS,
        WINDOW=WINDOW,
        TOPK=TOPK,
        S=S,
        BM=BM,
        dtype=_native.AFA_DTYPE[dtype],
        scale=SCALE,
        parts=parts,
        ring=ring,
        debug_rows=None if debug_rows is None else debug_rows.data_ptr(),
        softmax_lse=None if softmax_lse is None else softmax_lse.data_ptr(),
    )


def check_inputs(tensors, *, B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, TOPK, dtype, out_name="attention_out"):
    """Shape/dtype/device/contiguity contract of ``attention.py:211-224``."""
    b16 = DTYPES[dtype]
    i32 = torch.int32
    width = MAX_SEQ // PAGE
    shapes = {
        "q": ((T, H, D), b16),
        "ori_kv": ((ORI_BLOCKS, PAGE, 1, D), b16),
        "cmp_kv": ((CMP_BLOCKS, PAGE // RATIO, 1, D), b16),
        "cmp_sparse_indices": ((T, 1, TOPK), i32),
        "ori_block_table": ((B, width), i32),
        "cmp_block_table": ((B, width), i32),
        "cu_seqlens_q": ((B + 1,), i32),
        "seqused_ori_kv": ((B,), i32),
        "seqused_cmp_kv": ((B,), i32),
        "cmp_residual_kv": ((B,), i32),
        "ori_topk_length": ((T, 1), i32),
        "sinks": ((H,), torch.float32),
        out_name: ((T, H, D), b16),
    }
    device = None
    for name, tensor in tensors.items():
        shape, dt = shapes[name]
        check_tensor(name, tensor, shape, dt, device)
        device = tensor.device
    check_disjoint([(name, t, name == out_name) for name, t in tensors.items()])
    return device


TENSOR_NAMES = ("q", "ori_kv", "cmp_kv", "cmp_sparse_indices", "ori_block_table", "cmp_block_table", "cu_seqlens_q",
                "seqused_ori_kv", "seqused_cmp_kv", "cmp_residual_kv", "ori_topk_length", "sinks", "attention_out")


class Binding:
    """Launch state of one (device, stream, sizes) key, built and validated
    once: the launcher parameters, the workspace size and a reusable
    workspace. The counterpart of the reference runtime's ``KernelLaunch``,
    kept per (stream, runtime sizes) with its workspace allocated once
    (``src/runtime/torch.py:170-186``, ``src/runtime/kernel.py:39-50``).

    A later call with the same key checks each tensor's shape, dtype,
    contiguity and device in one pass and repeats the pairwise disjointness
    check only when a pointer differs from the last validated call."""

    __slots__ = ("device", "stream", "specs", "params", "params_ref", "nbytes", "workspace", "validated")

    def __init__(self, device, stream, specs, params, nbytes):
        self.device = device
        self.stream = stream
        self.specs = specs
        self.params = params
        self.params_ref = ct.pointer(params)
        self.nbytes = nbytes
        self.workspace = None
        self.validated = None


MAX_BINDINGS = 16
_bindings: "OrderedDict[tuple, Binding]" = OrderedDict()


def release_bindings():
    """Drops every cached binding and the workspaces they hold."""
    _bindings.clear()


def binding_key(device_index, stream, sizes):
    # The loaded library is part of the key: a binding's workspace size comes
    # from that library's workspace query (its split choice), so a binding
    # made through one library is never handed to another.
    return (id(_native.library()), device_index, stream) + sizes


def _binding(device, stream, sizes, policy, dtype, parts, ring):
    key = binding_key(device.index, stream, sizes)
    b = _bindings.get(key)
    if b is not None:
        _bindings.move_to_end(key)
        return b
    B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM, SCALE = policy
    b16 = DTYPES[dtype]
    i32 = torch.int32
    width = MAX_SEQ // PAGE
    shapes = ((T, H, D), (ORI_BLOCKS, PAGE, 1, D), (CMP_BLOCKS, PAGE // RATIO, 1, D), (T, 1, TOPK), (B, width),
              (B, width), (B + 1,), (B,), (B,), (B,), (T, 1), (H,), (T, H, D))
    dtypes = (b16, b16, b16, i32, i32, i32, i32, i32, i32, i32, i32, torch.float32, b16)
    specs = tuple((name, torch.Size(shape), dt) for name, shape, dt in zip(TENSOR_NAMES, shapes, dtypes))
    params = make_params(B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM, dtype, SCALE,
                         None, parts, None, ring)
    nbytes = ct.c_uint64(0)
    _native.check(_native.library().workspace_size_sparse_mla(ct.byref(nbytes), ct.byref(params)),
                  "workspace_size_sparse_mla")
    b = Binding(device, stream, specs, params, int(nbytes.value))
    _bindings[key] = b
    while len(_bindings) > MAX_BINDINGS:
        _bindings.popitem(last=False)
    return b


def _pointers(b, tensors):
    """Data pointers of the 13 operands after the per-call checks; any failure
    is reported by the full check (same messages as the first call)."""
    ptrs = []
    index = b.device.index
    for (name, shape, dt), t in zip(b.specs, tensors):
        if (not isinstance(t, torch.Tensor) or t.dtype is not dt or t.shape != shape or not t.is_contiguous()
                or t.get_device() != index):
            check_tensor(name, t, shape, dt, b.device)
        ptrs.append(t.data_ptr())
    return ptrs


def _prepare(
    q,
    ori_kv,
    cmp_kv,
    cmp_sparse_indices,
    ori_block_table,
    cmp_block_table,
    cu_seqlens_q,
    seqused_ori_kv,
    seqused_cmp_kv,
    cmp_residual_kv,
    ori_topk_length,
    sinks,
    attention_out,
    B=4,
    T=16,
    H=64,
    D=512,
    PAGE=128,
    RATIO=2,
    MAX_SEQ=4096,
    ORI_BLOCKS=128,
    CMP_BLOCKS=128,
    WINDOW=128,
    TOPK=512,
    ROWS=32,
    S=640,
    BM=64,
    PARTS=1,
    GROUPS=20,
    VR=16,
    BK=512,
    C=128,
    DTYPE="bf16",
    SCALE=0.04419417382415922,
    *,
    debug_rows=None,
    parts=None,
    softmax_lse=None,
    workspace=None,
    ring=None,
):
    """Validates one call and returns its launch state (see ``sparse_mla``)."""
    dtype = storage_dtype(DTYPE)
    tensors = (q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cmp_block_table, cu_seqlens_q, seqused_ori_kv,
               seqused_cmp_kv, cmp_residual_kv, ori_topk_length, sinks, attention_out)
    device_index = q.get_device() if isinstance(q, torch.Tensor) else -1
    if device_index < 0:
        check_tensor("q", q, (T, H, D), DTYPES[dtype])  # raises: not a device tensor
    stream = torch._C._cuda_getCurrentRawStream(device_index)
    sizes = (B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, ROWS, S, BM, PARTS, GROUPS, VR,
             BK, C, dtype, SCALE, parts, ring)
    b = _bindings.get(binding_key(device_index, stream, sizes))
    if b is None:
        check_policy(B, T, H, D, PAGE, RATIO, MAX_SEQ, WINDOW, TOPK, ROWS, S, BM, PARTS, GROUPS, VR, BK, C, SCALE)
        require(parts is None or parts in range(1, 9), "parts must be None or 1..8")
        require(ring in (None, 3, 4), "ring must be None, 3 or 4")
        check_inputs(
            dict(zip(TENSOR_NAMES, tensors)), B=B, T=T, H=H, D=D, PAGE=PAGE, RATIO=RATIO, MAX_SEQ=MAX_SEQ,
            ORI_BLOCKS=ORI_BLOCKS, CMP_BLOCKS=CMP_BLOCKS, TOPK=TOPK, dtype=dtype,
        )
        b = _binding(q.device, stream, sizes,
                     (B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM, SCALE),
                     dtype, parts or 0, ring or 0)
    ptrs = _pointers(b, tensors)
    params_ref = b.params_ref
    extra = ()
    if debug_rows is not None or softmax_lse is not None:
        # Per-call output pointers go into a copy, so the binding's parameters stay shared.
        params = SparseMlaParams.from_buffer_copy(b.params)
        if debug_rows is not None:
            check_tensor("debug_rows", debug_rows, (T, S, 2), torch.int32, b.device)
            params.debug_rows = debug_rows.data_ptr()
            extra += (("debug_rows", debug_rows),)
        if softmax_lse is not None:
            check_tensor("softmax_lse", softmax_lse, (T, H), torch.float32, b.device)
            params.softmax_lse = softmax_lse.data_ptr()
            extra += (("softmax_lse", softmax_lse),)
        params_ref = ct.pointer(params)
    own_workspace = workspace is None
    if workspace is not None:
        require(isinstance(workspace, torch.Tensor) and workspace.dtype == torch.uint8 and workspace.is_contiguous()
                and workspace.device == b.device, "workspace must be a contiguous uint8 tensor on the operands' device")
        require(workspace.numel() >= b.nbytes, f"workspace holds {workspace.numel()} bytes, needs {b.nbytes}")
        extra += (("workspace", workspace),)
    elif b.nbytes:
        if torch.cuda.is_current_stream_capturing():
            workspace = torch.empty(b.nbytes, dtype=torch.uint8, device=b.device)
        else:
            if b.workspace is None:
                b.workspace = torch.empty(b.nbytes, dtype=torch.uint8, device=b.device)
            workspace = b.workspace
    ws_ptr = None if workspace is None else workspace.data_ptr()
    signature = (*ptrs, ws_ptr, *((name, t.data_ptr(), t.numel()) for name, t in extra))
    if signature != b.validated:
        # Written operands (the output, the workspace, softmax_lse, the debug
        # image) must not overlap any other operand.
        named = [(name, t, name == "attention_out") for name, t in zip(TENSOR_NAMES, tensors)]
        named += [(name, t, True) for name, t in extra]
        if own_workspace and workspace is not None:
            named.append(("workspace", workspace, True))
        check_disjoint(named)
        b.validated = signature
    return device_index, stream, ptrs, ws_ptr, params_ref, workspace, attention_out


@functools.wraps(_prepare, assigned=("__module__",))
def sparse_mla(*args, **kwargs):
    """Sparse MLA forward; writes ``attention_out`` [T, H, D] and returns it.

    ``debug_rows`` (optional int32 [T, S, 2] device tensor) receives, per
    token, the compacted row list the kernel then streams: entry r < n is the
    r-th selected row as (cache, physical row), cache 0 = ori_kv,
    1 = cmp_kv, in slot order (window positions, then compressed ranks),
    and (-1, -1) from n on. With it the rows are resolved inside the
    attention kernel (one workgroup per token and head tile, no split).

    ``softmax_lse`` (optional float32 [T, H] device tensor) receives the
    natural-log normaliser ln(sum_j exp(s_j) + exp(sinks[h])) of every
    (token, head), i.e. the denominator of ``attention_out`` (the sink alone
    for an empty selection).

    ``parts`` (optional, 1..8) fixes how many workgroups share one token's
    selected rows on the plan path: 1 never splits, k > 1 splits every token
    into k parts whose partial results a merge kernel combines. By default only
    the tokens of an incomplete last round over the 256 CUs are split, where
    that shortens the longest per-CU stream (decode-sized batches).

    ``ring`` (optional, 3 or 4) fixes the KV ring of the persistent kernel on
    the plan path: 3 tiles of 32 rows (one chunk in flight) or 4 (two, where
    the row lists fit next to them). By default 4 when ``ori_kv`` and
    ``cmp_kv`` together exceed the 256 MiB Infinity Cache, else 3. The output
    does not depend on it.

    ``workspace`` (optional uint8 device tensor of at least
    ``workspace_bytes(...)`` bytes) replaces the binding's own workspace. When
    the plan path runs (at least two work items per CU, no split, no debug
    image), it holds the row-list plan afterwards (``plan_layout``): the
    selected-row count of every token, then every token's list of tagged
    rows (bit 31 set for cmp_kv) padded with its first row to whole 32-row
    chunks (32 entries of ori_kv row 0 for an empty selection).

    Without ``workspace``, each (device, stream, sizes) binding keeps one
    workspace and reuses it for every call on that stream (calls on one
    stream run in order); under HIP graph capture the call allocates its own
    from the graph's pool instead. ``release_bindings()`` frees them.
    """
    _, stream, ptrs, ws_ptr, params_ref, _, out = _prepare(*args, **kwargs)
    _native.check(_native.library().launch_sparse_mla(stream, *ptrs, ws_ptr, params_ref), "launch_sparse_mla")
    return out


def bind(*args, **kwargs):
    """Validates a ``sparse_mla`` call once and returns ``invoke()``, which
    launches it again on the current stream with no further checks (the
    reference's ``TensorKernel.bind``, ``src/runtime/torch.py:94-190``: bound
    tensors must keep their shape, dtype and storage). A stream other than the
    one current at bind time gets its own binding and workspace, as
    concurrent streams need separate bindings (``src/runtime/kernel.py:10``)."""
    device_index, stream0, ptrs, ws_ptr, params_ref, workspace, out = _prepare(*args, **kwargs)
    lib = _native.library()
    held = {stream0: (ptrs, ws_ptr, params_ref, workspace)}

    def invoke():
        stream = torch._C._cuda_getCurrentRawStream(device_index)
        state = held.get(stream)
        if state is None:
            _, _, p, w, r, ws, _ = _prepare(*args, **kwargs)
            state = held[stream] = (p, w, r, ws)
        _native.check(lib.launch_sparse_mla(stream, *state[0], state[1], state[2]), "launch_sparse_mla")
        return out

    return invoke


sparse_mla.bind = bind


def sparse_mla_planned(q, ori_kv, cmp_kv, sinks, attention_out, workspace, B, T, H=64, D=512, PAGE=128, RATIO=2,
                       MAX_SEQ=4096, ORI_BLOCKS=128, CMP_BLOCKS=128, WINDOW=128, TOPK=512, S=640, BM=64, DTYPE="bf16",
                       SCALE=0.04419417382415922, *, softmax_lse=None, ring=None):
    """The attention over a row-list plan alone (``launch_sparse_mla_planned``).

    ``workspace`` holds the plan of the same metadata and sizes, written by
    ``launch_sparse_mla_plan`` (``probe.sparse_mla_plan``; layout
    ``plan_layout``). Whether a plain ``sparse_mla`` call wrote a plan into its
    workspace depends on the device and the split, so that is not a plan to
    rely on; the kernel clamps every count and row id it reads to the list
    capacity and the caches, so a foreign workspace gives a wrong output, not
    a read outside ``ori_kv``/``cmp_kv``. Writes
    ``attention_out`` (and ``softmax_lse``) exactly as ``sparse_mla`` does on
    the same inputs, with the persistent kernel whatever ``T`` is, and returns
    it. ``ring`` as in ``sparse_mla``.
    """
    dtype = storage_dtype(DTYPE)
    require(BM in (32, 64) and H % BM == 0, "complete head tiles")
    require(D in (128, 256, 512), "gfx950 kernel supports D in {128, 256, 512}")
    require(ring in (None, 3, 4), "ring must be None, 3 or 4")
    b16 = DTYPES[dtype]
    device = q.device
    check_tensor("q", q, (T, H, D), b16, device)
    check_tensor("ori_kv", ori_kv, (ORI_BLOCKS, PAGE, 1, D), b16, device)
    check_tensor("cmp_kv", cmp_kv, (CMP_BLOCKS, PAGE // RATIO, 1, D), b16, device)
    check_tensor("sinks", sinks, (H,), torch.float32, device)
    check_tensor("attention_out", attention_out, (T, H, D), b16, device)
    _, rows_at, entries = plan_layout(T, WINDOW, TOPK)
    require(isinstance(workspace, torch.Tensor) and workspace.dtype == torch.uint8 and workspace.is_contiguous()
            and workspace.device == device, "workspace must be a contiguous uint8 tensor on the operands' device")
    require(workspace.numel() >= rows_at + 4 * T * entries, "workspace is smaller than the plan")
    named = [("q", q, False), ("ori_kv", ori_kv, False), ("cmp_kv", cmp_kv, False), ("sinks", sinks, False),
             ("workspace", workspace, False), ("attention_out", attention_out, True)]
    if softmax_lse is not None:
        check_tensor("softmax_lse", softmax_lse, (T, H), torch.float32, device)
        named.append(("softmax_lse", softmax_lse, True))
    check_disjoint(named)
    params = make_params(B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM, dtype, SCALE,
                         None, 1, softmax_lse, ring or 0)
    status = _native.library().launch_sparse_mla_planned(
        stream_handle(device), q.data_ptr(), ori_kv.data_ptr(), cmp_kv.data_ptr(), sinks.data_ptr(),
        attention_out.data_ptr(), workspace.data_ptr(), ct.byref(params))
    _native.check(status, "launch_sparse_mla_planned")
    return attention_out


def workspace_bytes(B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM, DTYPE="bf16",
                    SCALE=0.04419417382415922, parts=None):
    """Bytes of the optional workspace of one call (``workspace_size_sparse_mla``)."""
    params = make_params(B, T, H, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, BM,
                         storage_dtype(DTYPE), SCALE, None, parts or 0, None)
    nbytes = ct.c_uint64(0)
    _native.check(_native.library().workspace_size_sparse_mla(ct.byref(nbytes), ct.byref(params)),
                  "workspace_size_sparse_mla")
    return int(nbytes.value)


def plan_layout(T, WINDOW, TOPK):
    """Byte offsets of the row-list plan in the workspace: (counts offset,
    rows offset, entries per token). Counts are int32 [T] at offset 0; the
    row lists are uint32 [T][entries] from the 256-byte boundary after them,
    entries = WINDOW + TOPK rounded up to 256 (include/ascendflow_amd.h)."""
    counts = 0
    rows = -(-4 * T // 256) * 256
    return counts, rows, -(-(WINDOW + TOPK) // 256) * 256
