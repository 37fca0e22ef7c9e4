"""A seeded sweep of top-k selections against the oracle, bit for bit.

Crosses what the structured tests pin one at a time: row length (both
workgroup forms of the filter kernel: 256 threads up to 32K positions, 1024
beyond), TOPK, ratio, ragged request layouts with empty requests, and score
distributions chosen to stress the sampled threshold estimate (normal,
heavy ties, a tiny value range, constant blocks, mostly equal scores with a
few outliers, a sprinkling of +-inf and NaN).
"""

import numpy as np
import pytest
import torch

from ascendflow_amd.sparse_attention import sparse_topk_indices
from oracle import topk_reference as tr

pytestmark = pytest.mark.gpu

CASES = 30


def scores_for(rng, t, c, kind):
    if kind == "normal":
        return rng.normal(0.0, 1.0, (t, c)).astype(np.float32)
    if kind == "ties":
        return rng.integers(-3, 4, (t, c)).astype(np.float32)
    if kind == "narrow":
        return (1.0 + rng.integers(0, 64, (t, c)) * np.float32(2.0 ** -20)).astype(np.float32)
    if kind == "blocks":
        return np.repeat(rng.normal(0.0, 1.0, (t, -(-c // 97))), 97, axis=1)[:, :c].astype(np.float32)
    if kind == "outliers":
        s = np.zeros((t, c), np.float32)
        hot = rng.random((t, c)) < 0.002
        s[hot] = rng.normal(5.0, 1.0, int(hot.sum())).astype(np.float32)
        return s
    s = rng.normal(0.0, 1.0, (t, c)).astype(np.float32)  # "special"
    for value, share in ((np.inf, 0.001), (-np.inf, 0.01), (np.nan, 0.001)):
        s[rng.random((t, c)) < share] = value
    return s


def sweep_case(seed):
    rng = np.random.default_rng(seed)
    wide = rng.random() < 0.35
    c = int(rng.integers(32769, 70000)) if wide else int(rng.integers(1, 20000))
    b = int(rng.integers(1, 12))
    counts = rng.integers(0, 5, b).astype(np.int32)
    counts[rng.integers(b)] = max(1, int(counts.max()))
    ratio = int(rng.choice([1, 2]))
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    seq_cmp = rng.integers(0, c + 1, b).astype(np.int32)
    seq_cmp[rng.integers(b)] = c
    residual = (rng.integers(0, ratio, b) if ratio > 1 else np.zeros(b)).astype(np.int32)
    topk = int(rng.choice([1, 16, 512, 2048, 4000]))
    kind = str(rng.choice(["normal", "ties", "narrow", "blocks", "outliers", "special"]))
    return c, cu, seq_cmp, residual, topk, ratio, kind, rng


@pytest.mark.parametrize("seed", range(CASES))
def test_random_selection_matches_the_oracle(device, seed):
    c, cu, seq_cmp, residual, topk, ratio, kind, rng = sweep_case(seed)
    t = int(cu[-1])
    print(f"\n[topk sweep] seed={seed} C={c} B={len(seq_cmp)} T={t} TOPK={topk} R={ratio} scores={kind}", flush=True)
    scores = scores_for(rng, t, c, kind)
    to = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=device)
    buffer = torch.full((t * topk + 64,), 7, dtype=torch.int32, device=device)
    out = buffer[: t * topk].view(t, 1, topk)
    sparse_topk_indices(to(scores), to(cu), to(seq_cmp), to(residual), TOPK=topk, RATIO=ratio, out=out)
    torch.cuda.synchronize()
    assert torch.all(buffer[t * topk:] == 7), "write past the output"
    np.testing.assert_array_equal(out.cpu().numpy(), tr.topk_indices(scores, cu, seq_cmp, residual, topk, ratio))
