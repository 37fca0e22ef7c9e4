"""A seeded sweep of sparse-MLA configurations against the oracle.

The structured tests pin each feature on purpose-built inputs; this sweep
crosses them: random batch and token counts (the one-item kernel, the split
path and the plan + persistent path all occur), contexts, TOPK (one or
several 512-row blocks), D, heads per tile, ratio, dtype, the validation
case that generates the data, the persistent kernel's KV ring and the split
setting. Every case checks the output and softmax_lse against the FP32
oracle on sampled tokens, the guard words after the output, unchanged inputs,
and, when the plan path ran, the streamed plan bit for bit for every token.
"""

import numpy as np
import pytest
import torch

from oracle import sparse_reference as sr
from tests.sparse_helpers import assert_close, assert_plan_matches, call_args, call_kwargs, guard_intact, to_device

pytestmark = pytest.mark.gpu

LSE_RTOL, LSE_ATOL = 1e-4, 1e-3
CASES = 40


def sweep_case(seed):
    rng = np.random.default_rng(seed)
    d, h, bm = [(512, 64, 64), (512, 64, 32), (256, 64, 64), (256, 128, 64), (128, 32, 32), (128, 64, 32)][
        rng.integers(6)]
    b = int(rng.integers(1, 10))
    big = rng.random() < 0.5  # enough work items per CU for the plan + persistent path
    t = int(rng.integers(512 // (h // bm) + 8, 700)) if big else int(rng.integers(b, 4 * b + 40))
    t = max(t, b)
    max_seq = int(rng.choice([1024, 2048, 4096]))
    topk = int(rng.choice([1, 7, 64, 300, 512, 700, 1024]))
    blocks = b * (max_seq // 128) + int(rng.integers(0, 16))
    policy = sr.default_policy(B=b, T=t, H=h, D=d, BM=bm, MAX_SEQ=max_seq, TOPK=topk, ORI_BLOCKS=blocks,
                               CMP_BLOCKS=blocks, RATIO=int(rng.choice([1, 2])),
                               DTYPE=str(rng.choice(["bf16", "f16"])))
    policy["SCALE"] = d ** -0.5
    case = str(rng.choice(["mixed", "ragged", "padding", "duplicates", "replay", "sink", "window"]))
    ring = [None, 3, 4][rng.integers(3)]
    parts = [None, 1, 2, 3][rng.choice(4, p=[0.4, 0.3, 0.15, 0.15])]
    return policy, case, ring, parts


@pytest.mark.parametrize("seed", range(CASES))
def test_random_configuration_matches_the_oracle(device, seed):
    from ascendflow_amd.sparse_attention import sparse_mla
    from ascendflow_amd.sparse_attention.attention import workspace_bytes

    policy, case, ring, parts = sweep_case(seed)
    keys = ("B", "T", "H", "D", "BM", "MAX_SEQ", "TOPK", "RATIO", "DTYPE")
    print(f"\n[sweep] seed={seed} case={case} ring={ring} parts={parts} "
          + " ".join(f"{k}={policy[k]}" for k in keys), flush=True)
    data = sr.inputs(policy, case)
    tensors = to_device(data, policy, device)
    before = {k: tensors[k].clone() for k in sr.TENSOR_ORDER if k != "attention_out"}
    t = policy["T"]
    lse = torch.full((t, policy["H"]), float("nan"), dtype=torch.float32, device=device)
    size_keys = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW", "TOPK", "S",
                 "BM", "DTYPE", "SCALE")
    workspace = torch.full((workspace_bytes(**{k: policy[k] for k in size_keys}, parts=parts),), 0xCD,
                           dtype=torch.uint8, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), softmax_lse=lse, workspace=workspace, parts=parts,
               ring=ring)
    torch.cuda.synchronize()
    assert guard_intact(tensors), "kernel wrote past attention_out"
    for k, v in before.items():
        assert torch.equal(tensors[k], v), f"input {k} changed"
    out = tensors["attention_out"].float().cpu().numpy()
    assert np.isfinite(out).all(), "unwritten or non-finite output"
    rng = np.random.default_rng(1000 + seed)
    tokens = sorted({0, t - 1, *rng.choice(t, min(t, 20), replace=False).tolist()})
    assert_close(out[tokens], sr.oracle_fp32(data, policy, tokens), policy["DTYPE"])
    np.testing.assert_allclose(lse[torch.as_tensor(tokens, device=device)].cpu().numpy().astype(np.float64),
                               sr.oracle_lse(data, policy, tokens), rtol=LSE_RTOL, atol=LSE_ATOL)
    items = t * (policy["H"] // policy["BM"])
    if items >= 2 * 256 and parts in (None, 1):
        # The plan path (the split model only splits calls of at most one round).
        assert_plan_matches(workspace, data, policy, list(range(t)))
