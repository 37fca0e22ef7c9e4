"""HIP graph capture of the drop-in entries.

A serving loop can capture a step (top-k selection, sparse MLA, flash
attention) once and replay it, instead of launching every kernel from the
host each time. The entries launch only kernels on the current stream (no
allocation when the caller passes the workspace, no memset, no host sync), so
torch.cuda.graph captures them. Each test replays the captured graph several
times with eager work between the replays (the inputs rewritten in place with
new values, then a device synchronisation), and every replay must give the
bits an eager call gives on the same inputs.
"""

import pytest
import torch

from oracle import sparse_reference as sr
from tests.sparse_helpers import call_args, call_kwargs, guard_intact, to_device

pytestmark = pytest.mark.gpu

REPLAYS = 3


def capture(fn):
    """Warm fn up on a side stream (one-time library set-up stays out of the
    graph), then capture one call of it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def sparse_workspace(policy, device):
    from ascendflow_amd.sparse_attention.attention import workspace_bytes

    keys = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW", "TOPK", "S", "BM",
            "DTYPE", "SCALE")
    return torch.empty(workspace_bytes(**{k: policy[k] for k in keys}), dtype=torch.uint8, device=device)


def test_sparse_mla_graph_replays_match_eager(device):
    """B8 x T544 (at least two work items per CU: the plan kernel, then the
    persistent kernel) with a caller workspace and softmax_lse, captured once.
    Before each replay q and the sinks get new values; the replay's output and
    softmax_lse must equal an eager call's on the same inputs, bit for bit."""
    from ascendflow_amd.sparse_attention import sparse_mla

    print("\n[graph] sparse_mla B8 x T544", flush=True)
    policy = sr.default_policy(B=8, T=544, MAX_SEQ=4096, ORI_BLOCKS=160, CMP_BLOCKS=160)
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    kw = call_kwargs(policy)
    workspace = sparse_workspace(policy, device)
    lse = torch.full((policy["T"], policy["H"]), float("nan"), dtype=torch.float32, device=device)
    graph = capture(lambda: sparse_mla(*call_args(tensors), **kw, workspace=workspace, softmax_lse=lse))

    eager_out = torch.empty_like(tensors["attention_out"])
    eager_lse = torch.empty_like(lse)
    gen = torch.Generator(device=device)
    gen.manual_seed(20261202)
    for replay in range(REPLAYS):
        tensors["q"].copy_(torch.randn(tensors["q"].shape, generator=gen, device=device).mul_(0.5))
        tensors["sinks"].copy_(torch.randn(tensors["sinks"].shape, generator=gen, device=device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed, replayed_lse = tensors["attention_out"].clone(), lse.clone()
        assert torch.isfinite(replayed.float()).all(), f"replay {replay}: unwritten output"
        tensors["attention_out"].fill_(float("nan"))
        sparse_mla(*call_args(dict(tensors, attention_out=eager_out)), **kw, softmax_lse=eager_lse)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager_out), f"replay {replay} differs from the eager call"
        assert torch.equal(replayed_lse, eager_lse), f"replay {replay}: softmax_lse differs from the eager call"
        assert guard_intact(tensors), f"replay {replay} wrote past attention_out"


def test_topk_then_sparse_mla_graph_replays_match_eager(device):
    """The indexer chain captured as one graph: index scores ->
    sparse_topk_indices -> sparse_mla. Before each replay the scores get new
    values, so the selection (and the rows streamed) change; the replay's
    indices and output must equal the eager chain's."""
    from ascendflow_amd.sparse_attention import sparse_mla, sparse_topk_indices

    print("\n[graph] top-k -> sparse_mla B8 x T544", flush=True)
    policy = sr.default_policy(B=8, T=544, MAX_SEQ=4096, ORI_BLOCKS=160, CMP_BLOCKS=160)
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    kw = call_kwargs(policy)
    t, topk = policy["T"], policy["TOPK"]
    c = policy["MAX_SEQ"] // policy["RATIO"]
    scores = torch.empty((t, c), dtype=torch.float32, device=device)
    workspace = sparse_workspace(policy, device)
    indices = tensors["cmp_sparse_indices"]
    meta = (tensors["cu_seqlens_q"], tensors["seqused_cmp_kv"], tensors["cmp_residual_kv"])

    def chain(out_indices, out):
        sparse_topk_indices(scores, *meta, TOPK=topk, RATIO=policy["RATIO"], out=out_indices)
        sparse_mla(*call_args(dict(tensors, cmp_sparse_indices=out_indices, attention_out=out)), **kw,
                   workspace=workspace)

    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    scores.copy_(torch.randn(scores.shape, generator=gen, device=device))
    graph = capture(lambda: chain(indices, tensors["attention_out"]))
    eager_indices = torch.empty_like(indices)
    eager_out = torch.empty_like(tensors["attention_out"])
    previous = None
    for replay in range(REPLAYS):
        scores.copy_(torch.randn(scores.shape, generator=gen, device=device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed_indices, replayed = indices.clone(), tensors["attention_out"].clone()
        chain(eager_indices, eager_out)
        torch.cuda.synchronize()
        assert torch.equal(replayed_indices, eager_indices), f"replay {replay}: indices differ from the eager chain"
        assert torch.equal(replayed, eager_out), f"replay {replay}: output differs from the eager chain"
        if previous is not None:
            assert not torch.equal(previous, replayed_indices), "new scores did not change the selection"
        previous = replayed_indices
        assert guard_intact(tensors), f"replay {replay} wrote past attention_out"


@pytest.mark.parametrize("causal", [False, True])
def test_attention_target_graph_replays_match_eager(device, causal):
    """Flash attention (B1, H8/HKV2, Sq 1000, Sk 1500, f16): captured once,
    replayed with new Q/K/V values each time, equal to the eager call."""
    from ascendflow_amd.flash_attention import attention_target

    print(f"\n[graph] attention_target causal={causal}", flush=True)
    sq, sk = 1000, 1500
    q = torch.empty((1, 8, sq, 128), dtype=torch.float16, device=device)
    k = torch.empty((1, 2, sk, 128), dtype=torch.float16, device=device)
    v = torch.empty_like(k)
    out = torch.empty_like(q)
    eager = torch.empty_like(q)
    kw = dict(B=1, HQ=8, HKV=2, D=128, CAUSAL=causal)
    gen = torch.Generator(device=device)
    gen.manual_seed(11 + causal)
    for x in (q, k, v):
        x.copy_(torch.randn(x.shape, generator=gen, device=device))
    graph = capture(lambda: attention_target(q, k, v, out, sq, sk, **kw))
    for replay in range(REPLAYS):
        for x in (q, k, v):
            x.copy_(torch.randn(x.shape, generator=gen, device=device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        attention_target(q, k, v, eager, sq, sk, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(replayed.float()).all(), f"replay {replay}: non-finite output"
        assert torch.equal(replayed, eager), f"replay {replay} differs from the eager call"
