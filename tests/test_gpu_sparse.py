"""GPU parity of the fused sparse-MLA kernel against the CPU oracle.

Row selection is checked bit-exactly on the lists the kernels stream: the
plan workspace the persistent kernel reads (read back after the call), and
the one-item kernel's LDS row list (copied out through the debug image), plus
the per-slot gather image (the layout of the reference's gather workspace,
benchmarks/attention/run_sparse.py:111-130,253-262). Outputs are checked
against the FP32 oracle under the tolerance contract (max|err| <= 1e-2 *
max|ref|, plus the reference runner's rtol 0.02 / atol 0.005). Every case also
checks the 512 guard bytes after the output and that no input changed
(run_sparse.py:241-262 does the same on Ascend).
"""

import numpy as np
import pytest
import torch

from oracle import sparse_reference as sr
from tests.sparse_helpers import (INT_KEYS, assert_close, assert_plan_matches, call_args, call_kwargs, expected_rows,
                                  guard_intact, host_view, to_device)

pytestmark = pytest.mark.gpu

VARIANTS = {
    "bf16-d512-bm64-r2": dict(DTYPE="bf16", D=512, H=64, BM=64, RATIO=2),
    "bf16-d512-bm32-r2": dict(DTYPE="bf16", D=512, H=64, BM=32, RATIO=2),
    "f16-d256-bm64-r1": dict(DTYPE="f16", D=256, H=64, BM=64, RATIO=1),
    "bf16-d128-bm32-r2": dict(DTYPE="bf16", D=128, H=32, BM=32, RATIO=2),
    # A long selection: S = 3712, within the reference's resident capacity of
    # 4096 (attention.py:261); the LDS row list then holds 3712 entries.
    "bf16-d512-bm64-r2-topk3584": dict(DTYPE="bf16", D=512, H=64, BM=64, RATIO=2, TOPK=3584),
}


LSE_RTOL, LSE_ATOL = 1e-4, 1e-3  # FP32 scores from b16 inputs; exp2/log2 of the running sums


def assert_lse(actual, ref):
    actual = actual.cpu().numpy().astype(np.float64)
    assert np.isfinite(actual).all(), "non-finite softmax_lse"
    np.testing.assert_allclose(actual, ref, rtol=LSE_RTOL, atol=LSE_ATOL)


def run_case(policy, data, device):
    from ascendflow_amd.sparse_attention import sparse_mla, sparse_mla_gather

    tensors = to_device(data, policy, device)
    before = {k: tensors[k].clone() for k in sr.TENSOR_ORDER if k != "attention_out"}
    debug = torch.full((policy["T"], policy["S"], 2), -7, dtype=torch.int32, device=device)
    tensors["_lse"] = torch.full((policy["T"], policy["H"]), float("nan"), dtype=torch.float32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), debug_rows=debug, softmax_lse=tensors["_lse"])
    kv, bias = sparse_mla_gather(*(tensors[k] for k in ("ori_kv", "cmp_kv", *INT_KEYS)),
                                 **{k: policy[k] for k in ("B", "T", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS",
                                                           "CMP_BLOCKS", "WINDOW", "TOPK", "S", "DTYPE")})
    torch.cuda.synchronize()
    assert guard_intact(tensors), "kernel wrote past attention_out"
    for k, v in before.items():
        assert torch.equal(tensors[k], v), f"input {k} changed"
    assert_lse(tensors["_lse"], sr.oracle_lse(data, policy))
    return tensors, debug.cpu().numpy(), kv.float().cpu().numpy(), bias.cpu().numpy()


@pytest.mark.parametrize("variant", list(VARIANTS))
@pytest.mark.parametrize("case", sr.CASES)
def test_validation_cases_match_oracle(device, case, variant):
    print(f"\n[sparse] case={case} variant={variant}", flush=True)
    policy = sr.default_policy(B=4, T=16, MAX_SEQ=4096, ORI_BLOCKS=64, CMP_BLOCKS=64, **VARIANTS[variant])
    policy["SCALE"] = policy["D"] ** -0.5
    data = sr.inputs(policy, case)
    tensors, debug, kv, bias = run_case(policy, data, device)
    tokens = list(range(policy["T"]))
    np.testing.assert_array_equal(debug, expected_rows(data, policy, tokens))
    kv_ref, bias_ref = sr.gather_oracle(data, policy)
    np.testing.assert_array_equal(bias, bias_ref)
    np.testing.assert_array_equal(kv, kv_ref)
    actual = tensors["attention_out"].float().cpu().numpy()
    ref = sr.oracle_fp32(data, policy)
    assert_close(actual, ref, policy["DTYPE"])
    if case == "empty":
        assert np.all(actual == 0)
    # Without the debug image the call gets a plan workspace. With one part at
    # this size (fewer than two work items per CU) rows are still resolved
    # in-kernel: the same bits. By default (None) the library's cost model
    # splits each token of these small cases over several workgroups (far
    # fewer keys than CUs: one-item kernel on parts, then the merge kernel);
    # 2, 3 and 8 parts cover other merge widths, with masked placeholder parts
    # where a token has fewer chunks than parts.
    from ascendflow_amd.sparse_attention import sparse_mla

    fused = tensors["attention_out"].clone()
    fused_lse = tensors["_lse"].clone()
    lse_ref = sr.oracle_lse(data, policy)
    for parts in (1, None, 2, 3, 8):
        tensors["attention_out"].fill_(float("nan"))
        tensors["_lse"].fill_(float("nan"))
        sparse_mla(*call_args(tensors), **call_kwargs(policy), parts=parts, softmax_lse=tensors["_lse"])
        torch.cuda.synchronize()
        assert guard_intact(tensors), f"kernel wrote past attention_out (parts={parts})"
        if parts == 1:
            assert torch.equal(fused, tensors["attention_out"]), "the call without the debug image differs"
            assert torch.equal(fused_lse, tensors["_lse"]), "softmax_lse differs without the debug image"
            continue
        split = tensors["attention_out"].float().cpu().numpy()
        assert_close(split, ref, policy["DTYPE"])
        assert_lse(tensors["_lse"], lse_ref)
        if case == "empty":
            assert np.all(split == 0), f"empty selection not zero with parts={parts}"


PERSISTENT_VARIANTS = dict({v: VARIANTS[v] for v in VARIANTS if "topk" not in v},
                           # WINDOW + TOPK = 3712 slots: the plan kernel resolves a token in six
                           # sequences of round trips, and the persistent kernel's list ring holds
                           # 3840-entry lists (D = 256 leaves room for them next to the KV ring).
                           **{"bf16-d256-bm64-r2-topk3584": dict(DTYPE="bf16", D=256, H=64, BM=64, RATIO=2, TOPK=3584,
                                                                 MAX_SEQ=16384)})


def workspace_for(policy, device, parts=None):
    """A caller workspace for one call, filled with a sentinel so a plan the
    kernel did not write cannot pass for one."""
    from ascendflow_amd.sparse_attention.attention import workspace_bytes

    kw = {k: policy[k] for k in ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW",
                                 "TOPK", "S", "BM", "DTYPE", "SCALE")}
    return torch.full((workspace_bytes(**kw, parts=parts),), 0xCD, dtype=torch.uint8, device=device)


@pytest.mark.parametrize("ring", [3, 4])
@pytest.mark.parametrize("variant", list(PERSISTENT_VARIANTS))
def test_persistent_stream_matches_fused_and_oracle(device, variant, ring):
    """T = 544 tokens: at least two work items per CU, so the plan path runs
    the persistent kernel, whose workgroups stream many tokens (and, with
    BM = 32, both head tiles of a token) through one pipeline. With one part
    its output must equal the in-kernel row resolution bit for bit; with the
    tokens split over 2 or 4 workgroups (partial results merged, 3-tile ring)
    it must match the oracle on a sample that includes empty and one-row
    selections (the split runs on the one-item kernel, then the merge).
    ``ring``: the persistent kernel's KV ring of 3 or 4 tiles (one or two
    chunks in flight), whichever the automatic choice would take."""
    from ascendflow_amd.sparse_attention import sparse_mla

    print(f"\n[sparse] persistent stream variant={variant} ring={ring}", flush=True)
    policy = sr.default_policy(**dict(dict(B=6, T=544, MAX_SEQ=4096, ORI_BLOCKS=160, CMP_BLOCKS=160),
                                      **PERSISTENT_VARIANTS[variant]))
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    debug = torch.full((policy["T"], policy["S"], 2), -7, dtype=torch.int32, device=device)
    lse = torch.full((policy["T"], policy["H"]), float("nan"), dtype=torch.float32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), debug_rows=debug, softmax_lse=lse)
    torch.cuda.synchronize()
    fused, fused_lse = tensors["attention_out"].clone(), lse.clone()
    tensors["attention_out"].fill_(float("nan"))
    lse.fill_(float("nan"))
    workspace = workspace_for(policy, device, parts=1)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), parts=1, softmax_lse=lse, workspace=workspace, ring=ring)
    torch.cuda.synchronize()
    assert guard_intact(tensors), "kernel wrote past attention_out"
    assert torch.equal(fused, tensors["attention_out"]), "persistent stream differs from the in-kernel row resolution"
    assert torch.equal(fused_lse, lse), "persistent softmax_lse differs from the in-kernel row resolution"
    every = list(range(policy["T"]))
    assert_plan_matches(workspace, data, policy, every)
    np.testing.assert_array_equal(debug.cpu().numpy(), expected_rows(data, policy, every))
    rows = (debug[..., 0] >= 0).sum(dim=1).cpu().numpy()
    rng = np.random.default_rng(11)
    tokens = sorted({0, 1, 543, *np.flatnonzero(rows <= 1)[:8].tolist(), *rng.choice(544, 24, replace=False).tolist()})
    index = torch.as_tensor(tokens, device=device)
    ref = sr.oracle_fp32(data, policy, tokens)
    assert_close(tensors["attention_out"][index].float().cpu().numpy(), ref, policy["DTYPE"])
    lse_ref = sr.oracle_lse(data, policy, tokens)
    assert_lse(lse[index], lse_ref)
    for parts in (None, 2, 4):
        tensors["attention_out"].fill_(float("nan"))
        lse.fill_(float("nan"))
        sparse_mla(*call_args(tensors), **call_kwargs(policy), parts=parts, softmax_lse=lse)
        torch.cuda.synchronize()
        assert guard_intact(tensors), f"kernel wrote past attention_out (parts={parts})"
        assert torch.isfinite(tensors["attention_out"].float()).all(), f"unwritten output (parts={parts})"
        assert torch.isfinite(lse).all(), f"unwritten softmax_lse (parts={parts})"
        assert_close(tensors["attention_out"][index].float().cpu().numpy(), ref, policy["DTYPE"])
        assert_lse(lse[index], lse_ref)


@pytest.mark.parametrize("ring", [3, 4])
@pytest.mark.parametrize("variant", ["bf16-d512-bm64-r2", "f16-d256-bm64-r1"])
@pytest.mark.parametrize("case", sr.CASES)
def test_validation_cases_on_the_persistent_stream(device, case, variant, ring):
    """The eight validation cases (sparse_reference.py:45-104) at B8 x T544,
    i.e. more than two work items per CU, so the plain call takes the plan
    kernel + persistent kernel: empty selections, a ragged batch with an empty
    request, replay narrowing, padding, duplicates and sinks of +-80 all run
    through one continuous chunk stream per CU. The plan it streamed must equal
    the oracle's selection for every token, its output and softmax_lse must be
    bit-identical to the one-item kernel (whose own row list is checked through
    the debug image) and match the oracle on a sample. ``ring``: 3 or 4 KV
    ring tiles in the persistent kernel."""
    from ascendflow_amd.sparse_attention import sparse_mla

    print(f"\n[sparse] persistent case={case} variant={variant} ring={ring}", flush=True)
    policy = sr.default_policy(B=8, T=544, MAX_SEQ=4096, ORI_BLOCKS=160, CMP_BLOCKS=160, **VARIANTS[variant])
    policy["SCALE"] = policy["D"] ** -0.5
    data = sr.inputs(policy, case)
    tensors = to_device(data, policy, device)
    before = {k: tensors[k].clone() for k in sr.TENSOR_ORDER if k != "attention_out"}
    t = policy["T"]
    debug = torch.full((t, policy["S"], 2), -7, dtype=torch.int32, device=device)
    lse_one = torch.full((t, policy["H"]), float("nan"), dtype=torch.float32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), debug_rows=debug, softmax_lse=lse_one)
    torch.cuda.synchronize()
    one_item = tensors["attention_out"].clone()
    tensors["attention_out"].fill_(float("nan"))
    lse = torch.full_like(lse_one, float("nan"))
    workspace = workspace_for(policy, device, parts=1)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), parts=1, softmax_lse=lse, workspace=workspace, ring=ring)
    torch.cuda.synchronize()
    assert guard_intact(tensors), "kernel wrote past attention_out"
    for k, v in before.items():
        assert torch.equal(tensors[k], v), f"input {k} changed"
    every = list(range(t))
    assert_plan_matches(workspace, data, policy, every)
    np.testing.assert_array_equal(debug.cpu().numpy(), expected_rows(data, policy, every))
    assert torch.equal(one_item, tensors["attention_out"]), "persistent stream differs from the one-item kernel"
    assert torch.equal(lse_one, lse), "persistent softmax_lse differs from the one-item kernel"
    out = tensors["attention_out"].float().cpu().numpy()
    if case == "empty":
        assert np.all(out == 0)
    counts = (debug[..., 0] >= 0).sum(dim=1).cpu().numpy()
    rng = np.random.default_rng(3)
    tokens = sorted({0, 1, t - 1, *np.flatnonzero(counts <= 1)[:6].tolist(), *np.flatnonzero(counts == counts.max())[:2].tolist(),
                     *rng.choice(t, 24, replace=False).tolist()})
    assert_close(out[tokens], sr.oracle_fp32(data, policy, tokens), policy["DTYPE"])
    assert_lse(lse[torch.as_tensor(tokens, device=device)], sr.oracle_lse(data, policy, tokens))


@pytest.mark.parametrize("ring", [3, 4])
@pytest.mark.parametrize("variant", ["bf16-d512-bm64-r2", "bf16-d512-bm32-r2"])
@pytest.mark.parametrize("case", sr.CASES)
def test_persistent_stream_with_few_tokens_per_request(device, case, variant, ring):
    """B40 x T560 (14 query tokens per request on average): more than two work
    items per CU, so the plan path runs the persistent kernel, and at most 16
    tokens per request, so at D = 512 it takes its form with non-temporal KV,
    Q and O accesses (the batched-decode form). On each of the eight
    validation cases its output and softmax_lse must be bit-identical to the
    one-item kernel's, its plan must equal the oracle's selection, and a
    sample must match the oracle (all zero for empty selections); both KV
    rings, one and two head tiles per token."""
    from ascendflow_amd.sparse_attention import sparse_mla

    print(f"\n[sparse] persistent few-token case={case} variant={variant} ring={ring}", flush=True)
    policy = sr.default_policy(B=40, T=560, MAX_SEQ=4096, ORI_BLOCKS=160, CMP_BLOCKS=160, **VARIANTS[variant])
    policy["SCALE"] = policy["D"] ** -0.5
    data = sr.inputs(policy, case)
    tensors = to_device(data, policy, device)
    t = policy["T"]
    debug = torch.full((t, policy["S"], 2), -7, dtype=torch.int32, device=device)
    lse_one = torch.full((t, policy["H"]), float("nan"), dtype=torch.float32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), debug_rows=debug, softmax_lse=lse_one)
    torch.cuda.synchronize()
    one_item = tensors["attention_out"].clone()
    tensors["attention_out"].fill_(float("nan"))
    lse = torch.full_like(lse_one, float("nan"))
    workspace = workspace_for(policy, device, parts=1)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), parts=1, softmax_lse=lse, workspace=workspace, ring=ring)
    torch.cuda.synchronize()
    assert guard_intact(tensors), "kernel wrote past attention_out"
    every = list(range(t))
    assert_plan_matches(workspace, data, policy, every)
    np.testing.assert_array_equal(debug.cpu().numpy(), expected_rows(data, policy, every))
    assert torch.equal(one_item, tensors["attention_out"]), "persistent stream differs from the one-item kernel"
    assert torch.equal(lse_one, lse), "persistent softmax_lse differs from the one-item kernel"
    counts = (debug[..., 0] >= 0).sum(dim=1).cpu().numpy()
    rng = np.random.default_rng(5)
    tokens = sorted({0, 1, t - 1, *np.flatnonzero(counts <= 1)[:6].tolist(), *rng.choice(t, 24, replace=False).tolist()})
    out = tensors["attention_out"].float().cpu().numpy()
    if case == "empty":
        assert np.all(out == 0)
    assert_close(out[tokens], sr.oracle_fp32(data, policy, tokens), policy["DTYPE"])
    assert_lse(lse[torch.as_tensor(tokens, device=device)], sr.oracle_lse(data, policy, tokens))


@pytest.mark.parametrize("shape,ring", [("b8-t544", 3), ("b8-t544", 4), ("b40-t560", 3), ("b40-t560", 4), ("b4-t16", None)])
def test_plan_then_planned_attention_equals_the_call(device, shape, ring):
    """launch_sparse_mla_plan followed by launch_sparse_mla_planned (the
    persistent kernel alone over that plan) gives sparse_mla's output and
    softmax_lse bit for bit: at T544 (where sparse_mla itself takes the plan
    path; each KV ring), at B40 x T560 (14 tokens per request: the plan path
    with the persistent kernel's non-temporal form) and at T16 (where it runs
    the one-item kernel, whose output the persistent kernel matches bit for
    bit when no key is split: parts=1, and the planned call still runs the
    persistent kernel)."""
    from ascendflow_amd.sparse_attention import sparse_mla, sparse_mla_planned
    from ascendflow_amd.sparse_attention.probe import sparse_mla_plan

    print(f"\n[sparse] plan + planned {shape} ring={ring}", flush=True)
    b, t = {"b8-t544": (8, 544), "b40-t560": (40, 560), "b4-t16": (4, 16)}[shape]
    policy = sr.default_policy(B=b, T=t, MAX_SEQ=4096, ORI_BLOCKS=160, CMP_BLOCKS=160)
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    lse = torch.full((t, policy["H"]), float("nan"), dtype=torch.float32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), softmax_lse=lse, parts=1)
    torch.cuda.synchronize()
    whole, whole_lse = tensors["attention_out"].clone(), lse.clone()
    tensors["attention_out"].fill_(float("nan"))
    lse.fill_(float("nan"))
    workspace = sparse_mla_plan(tensors, policy)
    sparse_mla_planned(*(tensors[k] for k in ("q", "ori_kv", "cmp_kv", "sinks", "attention_out")), workspace,
                       **call_kwargs(policy), softmax_lse=lse, ring=ring)
    torch.cuda.synchronize()
    assert guard_intact(tensors), "kernel wrote past attention_out"
    assert torch.equal(whole, tensors["attention_out"]), "plan + planned attention differs from the call"
    assert torch.equal(whole_lse, lse), "plan + planned softmax_lse differs from the call"


def test_relaunch_is_bitwise_deterministic(device):
    from ascendflow_amd.sparse_attention import sparse_mla

    policy = sr.default_policy(B=4, T=16, MAX_SEQ=4096, ORI_BLOCKS=64, CMP_BLOCKS=64)
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy))
    first = tensors["attention_out"].clone()
    for _ in range(3):
        sparse_mla(*call_args(tensors), **call_kwargs(policy))
    torch.cuda.synchronize()
    assert torch.equal(first, tensors["attention_out"])


def test_binding_reuse_bind_and_streams_give_the_same_output(device):
    """The per-(device, stream, sizes) binding: a first call builds it, later
    calls reuse its parameters and workspace; ``sparse_mla.bind`` validates
    once and relaunches; another stream gets its own binding. On the plan +
    persistent path (T = 544 over 8 requests) every variant must give the
    first call's output and softmax_lse bit for bit."""
    from ascendflow_amd.sparse_attention import attention as A
    from ascendflow_amd.sparse_attention import sparse_mla

    A.release_bindings()
    policy = sr.default_policy(B=8, T=544, MAX_SEQ=4096, ORI_BLOCKS=256, CMP_BLOCKS=256)
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    lse = torch.empty((policy["T"], policy["H"]), dtype=torch.float32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), softmax_lse=lse)
    torch.cuda.synchronize()
    first, first_lse = tensors["attention_out"].clone(), lse.clone()
    assert len(A._bindings) == 1
    binding = next(iter(A._bindings.values()))
    assert binding.workspace is not None and binding.workspace.numel() == binding.nbytes
    for _ in range(2):
        tensors["attention_out"].zero_()
        sparse_mla(*call_args(tensors), **call_kwargs(policy), softmax_lse=lse)
    torch.cuda.synchronize()
    assert len(A._bindings) == 1
    assert torch.equal(first, tensors["attention_out"]) and torch.equal(first_lse, lse)
    invoke = sparse_mla.bind(*call_args(tensors), **call_kwargs(policy), softmax_lse=lse)
    tensors["attention_out"].zero_()
    lse.zero_()
    invoke()
    torch.cuda.synchronize()
    assert torch.equal(first, tensors["attention_out"]) and torch.equal(first_lse, lse)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        tensors["attention_out"].zero_()
        invoke()
        sparse_mla(*call_args(tensors), **call_kwargs(policy))
    torch.cuda.synchronize()
    assert len(A._bindings) == 2  # one more binding: the side stream's (its bound and plain calls share it)
    assert torch.equal(first, tensors["attention_out"])
    assert guard_intact(tensors), "kernel wrote past attention_out"
    A.release_bindings()


def test_written_operands_must_not_overlap_the_workspace(device):
    """softmax_lse or the debug image carved out of the caller's workspace is
    rejected before any launch (the plan would otherwise overwrite them, or
    they the plan)."""
    from ascendflow_amd.sparse_attention import sparse_mla

    policy = sr.default_policy(B=8, T=544, MAX_SEQ=4096, ORI_BLOCKS=256, CMP_BLOCKS=256)
    tensors = to_device(sr.inputs(policy, "mixed"), policy, device)
    workspace = workspace_for(policy, device)
    lse = workspace[: policy["T"] * policy["H"] * 4].view(torch.float32).view(policy["T"], policy["H"])
    with pytest.raises(ValueError, match="overlap"):
        sparse_mla(*call_args(tensors), **call_kwargs(policy), softmax_lse=lse, workspace=workspace)
    # A debug image that starts in the workspace's last 256 bytes.
    debug_bytes = policy["T"] * policy["S"] * 8
    big = torch.empty(workspace.numel() + debug_bytes, dtype=torch.uint8, device=device)
    debug = big[workspace.numel() - 256 : workspace.numel() - 256 + debug_bytes].view(torch.int32)
    debug = debug.view(policy["T"], policy["S"], 2)
    with pytest.raises(ValueError, match="overlap"):
        sparse_mla(*call_args(tensors), **call_kwargs(policy), debug_rows=debug, workspace=big[: workspace.numel()])
    out_alias = tensors["attention_out"].view(torch.uint8).view(-1)[: workspace.numel()]
    if out_alias.numel() == workspace.numel():
        with pytest.raises(ValueError, match="overlap"):
            sparse_mla(*call_args(tensors), **call_kwargs(policy), workspace=out_alias)


def metadata_view(inputs):
    """The integer metadata of device-built inputs as an oracle data dict (no rows)."""
    return {k: inputs.host[k] for k in INT_KEYS}


def check_measured(inputs, tokens, device, split=False, plan=False):
    """Runs without the debug image first (the path the benchmark takes), then
    with it (in-kernel row resolution, one part per token). Unless the plan
    path splits tokens into parts (``split``: the merge sums in another
    order), the debug dump must not change any output bit; both outputs must
    match the oracle on ``tokens``. The debug image (the one-item kernel's
    streamed row list) must equal the oracle's selection for every token; with
    ``plan`` the plain call ran the plan + persistent path, and the plan it
    streamed (read back from the workspace) must too, and forcing either KV
    ring of the persistent kernel (3 or 4 tiles) must not change a bit."""
    from ascendflow_amd.sparse_attention import sparse_mla

    policy = inputs.policy
    workspace = workspace_for(policy, device)
    sparse_mla(*inputs.call_args(), **inputs.call_kwargs(), workspace=workspace)
    torch.cuda.synchronize()
    plain = inputs.tensors["attention_out"].clone()
    every = list(range(policy["T"]))
    meta = metadata_view(inputs)
    if plan:
        assert_plan_matches(workspace, meta, policy, every)
        for ring in (3, 4):
            sparse_mla(*inputs.call_args(), **inputs.call_kwargs(), workspace=workspace, ring=ring)
            torch.cuda.synchronize()
            assert torch.equal(plain, inputs.tensors["attention_out"]), f"ring {ring} changed the output"
    del workspace
    debug = torch.full((policy["T"], policy["S"], 2), -7, dtype=torch.int32, device=device)
    sparse_mla(*inputs.call_args(), **inputs.call_kwargs(), debug_rows=debug)
    torch.cuda.synchronize()
    if not split:
        assert torch.equal(plain, inputs.tensors["attention_out"]), "the debug image changed the output"
    for first in range(0, policy["T"], 4096):
        part = every[first : first + 4096]
        np.testing.assert_array_equal(debug[first : first + len(part)].cpu().numpy(), expected_rows(meta, policy, part))
    del debug
    data = host_view(inputs, tokens)
    index = torch.as_tensor(tokens, device=device)
    ref = sr.oracle_fp32(data, policy, tokens)
    assert_close(plain[index].float().cpu().numpy(), ref, policy["DTYPE"])
    actual = inputs.tensors["attention_out"][index].float().cpu().numpy()
    return assert_close(actual, ref, policy["DTYPE"])


def test_decode_b64x6_ctx128k_all_tokens(device):
    """Decode configuration: every one of the 384 tokens."""
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print("\n[sparse] decode B64x6 ctx 131072", flush=True)
    policy = measurement_policy(batch=64, query_tokens=6, context=131072)
    inputs = make_inputs(policy, 131072, device=device)
    check_measured(inputs, list(range(policy["T"])), device)
    # Forced split: every token over two workgroups, partial results merged.
    from ascendflow_amd.sparse_attention import sparse_mla

    plain = inputs.tensors["attention_out"].clone()
    sparse_mla(*inputs.call_args(), **inputs.call_kwargs(), parts=2)
    torch.cuda.synchronize()
    split = inputs.tensors["attention_out"].float()
    err = (split - plain.float()).abs().max().item()
    assert err <= 1e-2 * plain.float().abs().max().item(), f"split decode differs by {err}"



@pytest.mark.parametrize("per_request", [16, 17])
def test_decode_either_side_of_the_streaming_kv_threshold(device, per_request):
    """The one-item kernel loads KV rows non-temporally for calls of at most 16
    query tokens per request (T <= 16 B) and with ordinary loads above: both
    instantiations (D = 512) match the oracle on every token, with the keys
    split automatically (these calls fill less than one round of CUs) and
    whole."""
    from ascendflow_amd.sparse_attention import sparse_mla
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print(f"\n[sparse] B2 x {per_request} ctx 8192", flush=True)
    policy = measurement_policy(batch=2, query_tokens=per_request, context=8192)
    inputs = make_inputs(policy, 8192, device=device)
    tokens = list(range(policy["T"]))
    check_measured(inputs, tokens, device, split=True)
    sparse_mla(*inputs.call_args(), **inputs.call_kwargs(), parts=1)
    torch.cuda.synchronize()
    assert_close(inputs.tensors["attention_out"].float().cpu().numpy(),
                 sr.oracle_fp32(host_view(inputs, tokens), policy, tokens), policy["DTYPE"])


@pytest.mark.parametrize("batch", [1, 4, 48])
def test_decode_small_batches_split_automatically(device, batch):
    """Decode with few requests (x 6 queries at 128K): the library splits the
    keys beyond the last full round of 256 into parts (B1 and B4: every key,
    7 and 5 parts; B48: the 32 keys after a full round, 5 parts, launched
    after the whole keys and mapped to XCDs as their own segment) and merges
    them. Outputs and softmax_lse must match the oracle on a sample covering
    whole and split keys; the debug call (no split) must agree within the
    same tolerance and select the oracle's rows."""
    from ascendflow_amd.sparse_attention import sparse_mla
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print(f"\n[sparse] decode B{batch}x6 ctx 131072 (automatic split)", flush=True)
    policy = measurement_policy(batch=batch, query_tokens=6, context=131072)
    inputs = make_inputs(policy, 131072, device=device)
    T = policy["T"]
    rng = np.random.default_rng(batch)
    tokens = sorted({0, T - 1, *rng.choice(T, min(T, 24), replace=False).tolist()}
                    | ({255, 256, 257, 270, 287} if T > 256 else set()))
    check_measured(inputs, tokens, device, split=True)
    lse = torch.full((T, policy["H"]), float("nan"), dtype=torch.float32, device=device)
    sparse_mla(*inputs.call_args(), **inputs.call_kwargs(), softmax_lse=lse)
    torch.cuda.synchronize()
    data = host_view(inputs, tokens)
    index = torch.as_tensor(tokens, device=device)
    assert_lse(lse[index], sr.oracle_lse(data, policy, tokens))
    assert_close(inputs.tensors["attention_out"][index].float().cpu().numpy(), sr.oracle_fp32(data, policy, tokens),
                 policy["DTYPE"])


def test_prefill_q8k_ctx32k_sampled_tokens(device):
    """Prefill configuration on a spread sample of tokens."""
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print("\n[sparse] prefill T8192 ctx 32768", flush=True)
    policy = measurement_policy(batch=1, query_tokens=8192, context=32768)
    inputs = make_inputs(policy, 32768, device=device)
    rng = np.random.default_rng(5)
    tokens = sorted({0, 1, 31, 32, 8191, *rng.choice(8192, 90, replace=False).tolist()})
    check_measured(inputs, tokens, device, plan=True)


def test_prefill_q32k_ctx32k_all_rows_and_sampled_tokens(device):
    """Prefill at scale (README.md:34): B1, Q 32768 tokens
    over a 32K context, so selections grow from 1 row (token 0) to 640. The
    plan + persistent path streams 128 work items per CU over a 100 MB plan:
    its lists must equal the oracle's selection for all 32768 tokens, its
    output must be bit-identical to the one-item kernel's (whose row lists
    are checked for every token through the debug image) and match the FP32
    oracle on spread tokens, including both ends and chunk/half boundaries."""
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print("\n[sparse] prefill T32768 ctx 32768", flush=True)
    policy = measurement_policy(batch=1, query_tokens=32768, context=32768)
    inputs = make_inputs(policy, 32768, device=device)
    rng = np.random.default_rng(32)
    tokens = sorted({0, 1, 31, 32, 63, 64, 255, 256, 1023, 8191, 8192, 16383, 16384, 32766, 32767,
                     *rng.choice(32768, 90, replace=False).tolist()})
    check_measured(inputs, tokens, device, plan=True)


def test_prefill_from_empty_cache_has_growing_selections(device):
    """Q = context: early tokens have short windows and few compressed rows."""
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print("\n[sparse] prefill T4096 ctx 4096", flush=True)
    policy = measurement_policy(batch=1, query_tokens=4096, context=4096)
    inputs = make_inputs(policy, 4096, device=device)
    tokens = list(range(0, 40)) + list(range(100, 4096, 97)) + [4095]
    check_measured(inputs, tokens, device, plan=True)


def test_decode_b128x6_ctx128k_sampled_tokens(device):
    """The reference README's second decode row (B128 x 6 queries = 768 tokens
    at 128K, README.md:36): three full rounds of 256 work items, no split."""
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    print("\n[sparse] decode B128x6 ctx 131072", flush=True)
    policy = measurement_policy(batch=128, query_tokens=6, context=131072)
    inputs = make_inputs(policy, 131072, device=device)
    rng = np.random.default_rng(7)
    tokens = sorted({0, 5, 6, 767, *rng.choice(768, 60, replace=False).tolist()})
    check_measured(inputs, tokens, device, plan=True)


@pytest.mark.parametrize("variant", ["bf16-d512-bm64-r2", "f16-d256-bm64-r1", "bf16-d128-bm32-r2"])
def test_framework_op_matches_entry_and_oracle(device, variant):
    """torch.ops.ascendflow_amd.sparse_flash_mla (vendor-operator call
    convention, sizes from shapes, output and LSE allocated) gives the same
    bits as the drop-in entry and matches the oracle, LSE included."""
    import ascendflow_amd.sparse_attention  # noqa: F401  registers the op
    from ascendflow_amd.sparse_attention import sparse_mla

    policy = sr.default_policy(B=4, T=16, MAX_SEQ=4096, ORI_BLOCKS=64, CMP_BLOCKS=64, **VARIANTS[variant])
    policy["SCALE"] = policy["D"] ** -0.5
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    args = [tensors[k] for k in sr.TENSOR_ORDER if k != "attention_out"]
    out, lse = torch.ops.ascendflow_amd.sparse_flash_mla(*args, policy["SCALE"], policy["RATIO"],
                                                         ori_win_left=policy["WINDOW"] - 1, return_softmax_lse=True)
    entry_lse = torch.empty_like(lse)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), softmax_lse=entry_lse)
    torch.cuda.synchronize()
    assert torch.equal(out, tensors["attention_out"]), "framework op differs from sparse_mla"
    assert torch.equal(lse, entry_lse), "framework op softmax_lse differs from sparse_mla"
    assert_close(out.float().cpu().numpy(), sr.oracle_fp32(data, policy), policy["DTYPE"])
    assert_lse(lse, sr.oracle_lse(data, policy))
    out2, empty = torch.ops.ascendflow_amd.sparse_flash_mla(*args, policy["SCALE"], policy["RATIO"],
                                                            ori_win_left=policy["WINDOW"] - 1)
    torch.cuda.synchronize()
    assert empty.numel() == 0 and torch.equal(out2, out)
    with pytest.raises(ValueError):
        torch.ops.ascendflow_amd.sparse_flash_mla(*args, policy["SCALE"], policy["RATIO"], ori_mask_mode=1)


def test_plan_entry_and_gather_probe_on_decode(device):
    """launch_sparse_mla_plan writes the oracle's selection for all 384 decode
    tokens (B64 x 6 at 128K), and the gather probe streams exactly the planned
    rows at every depth, interleaved and balanced (its checksum of the first
    dword of every streamed row equals torch's)."""
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy
    from ascendflow_amd.sparse_attention.probe import expected_probe_sum, gather_probe, sparse_mla_plan

    print("\n[sparse] plan entry + gather probe, decode B64x6 ctx 131072", flush=True)
    policy = measurement_policy(batch=64, query_tokens=6, context=131072)
    inputs = make_inputs(policy, 131072, device=device)
    workspace = sparse_mla_plan(inputs.tensors, policy)
    torch.cuda.synchronize()
    assert_plan_matches(workspace, metadata_view(inputs), policy, list(range(policy["T"])))
    want = expected_probe_sum(inputs.tensors, policy, workspace)
    for depth in (1, 2, 4, 6, 8):
        for grid, balanced in ((384, False), (256, False), (256, True)):
            sums = gather_probe(inputs.tensors, policy, workspace, grid, depth, balanced)
            torch.cuda.synchronize()
            got = int(sums.long().sum().item()) & 0xFFFFFFFF
            assert got == want, f"probe depth {depth} grid {grid} balanced {balanced}: checksum {got:#x} != {want:#x}"
