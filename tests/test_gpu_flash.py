"""GPU parity of the flash-attention and teaching-attention kernels against the CPU oracle.

Flash attention is checked the way the reference's runner checks it
(benchmarks/attention/run.py:606-707, benchmarks/validation/attention.py:60-121):
against the FP32 online recurrence (P rounded before PV) with the KV blocking
of the host policy (causal_policy's kv_tile), on the reference's data cases
(standard, uniform K, sharp Q/K at N(0,1)*0.5) and sampled rows {0, 7, 63, 64,
71, 127} of every 128-row query tile plus the last row, at the contract's
tolerance: f16 rtol 0.002 / atol 0.0002, bf16 rtol 0.01 / atol 0.001
(benchmarks/attention/contract.py:121-122), as allclose(actual, expected).
The BASELINE bar max|err| <= 1e-2 * max|ref| against dense FP32 softmax is
checked as well.
"""

import numpy as np
import pytest
import torch

from oracle.attention import dense_reference, inputs, online_attention, simple_reference
from oracle.dtypes import rounded

pytestmark = pytest.mark.gpu

TORCH = {"f16": torch.float16, "bf16": torch.bfloat16}
TOLERANCE = {"f16": (0.002, 0.0002), "bf16": (0.01, 0.001)}  # contract.py:121-122


def sampled_rows(sq):
    """Rows {0, 7, 63, 64, 71, 127} of every 128-row tile, plus the last row
    (benchmarks/validation/attention.py:91-104)."""
    rows = {t * 128 + r for t in range(-(-sq // 128)) for r in (0, 7, 63, 64, 71, 127) if t * 128 + r < sq}
    return np.array(sorted(rows | {sq - 1}), np.int64)


def kv_tile(sq, sk):
    from ascendflow_amd.flash_attention import causal_policy

    return causal_policy(sq, sk)["kv_tile"]


def online_rows(q, k, v, rows, dtype, causal, block_kv):
    """Oracle output of query rows ``rows`` for every (batch, head) [B, HQ, len(rows), D]."""
    b, hq = q.shape[:2]
    group = hq // k.shape[1]
    out = np.empty((b, hq, len(rows), q.shape[-1]), np.float32)
    for bi in range(b):
        for h in range(hq):
            for first in range(0, len(rows), 128):
                part = rows[first : first + 128]
                out[bi, h, first : first + len(part)] = online_attention(
                    q[bi, h, part], k[bi, h // group], v[bi, h // group], block_kv=block_kv, dtype=dtype,
                    scale=np.float32(1 / np.sqrt(128)), causal=causal, query_positions=part)
    return out


def assert_contract(actual, expected, dtype):
    """The reference runner's check: finite, then allclose at the contract tolerance."""
    assert np.isfinite(actual).all(), "non-finite or unwritten attention output"
    rtol, atol = TOLERANCE[dtype]
    err = float(np.max(np.abs(actual - expected)))
    assert np.allclose(actual, expected, rtol=rtol, atol=atol), (
        f"attention output differs from the online oracle at rtol {rtol} / atol {atol}; max|err| {err:.3g}")


def assert_baseline_bar(actual, ref):
    err = float(np.max(np.abs(actual - ref)))
    bound = 1e-2 * float(np.max(np.abs(ref)))
    assert err <= bound, f"max|err| {err:.3g} > 1e-2 * max|ref| = {bound:.3g}"


def run_fa(data, dtype, causal, device, **kw):
    from ascendflow_amd.flash_attention import attention_target

    q, k, v = (torch.from_numpy(data[n]).to(device, TORCH[dtype]) for n in ("q", "k", "v"))
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    guarded = torch.full((q.numel() + 256,), float("nan"), dtype=q.dtype, device=device)
    o = guarded[: q.numel()].view(q.shape)
    attention_target(q, k, v, o, sq, sk, B=b, HQ=hq, HKV=hkv, D=d, DTYPE=dtype, SCALE=d**-0.5, CAUSAL=causal, **kw)
    torch.cuda.synchronize()
    assert torch.isnan(guarded[q.numel():].float()).all(), "kernel wrote past O"
    for name, tensor in (("q", q), ("k", k), ("v", v)):
        assert torch.equal(tensor.float().cpu(), torch.from_numpy(data[name])), f"input {name} changed"
    return o.float().cpu().numpy()


@pytest.mark.parametrize(
    "b,hq,hkv,sq,sk,dtype,causal,case",
    [
        (1, 8, 8, 2048, 2048, "f16", False, "standard"),
        (1, 8, 8, 2048, 2048, "f16", False, "sharp"),
        (1, 8, 8, 2048, 2048, "f16", False, "uniform"),
        (1, 8, 8, 2048, 2048, "f16", True, "standard"),
        (1, 8, 8, 2048, 2048, "f16", True, "sharp"),
        (1, 8, 2, 1024, 4096, "bf16", False, "standard"),
        (1, 8, 2, 1024, 4096, "bf16", True, "sharp"),
        (2, 8, 2, 300, 700, "bf16", False, "standard"),
        (2, 8, 2, 300, 700, "bf16", True, "standard"),
        (1, 4, 1, 700, 300, "f16", True, "standard"),
        (1, 4, 1, 700, 300, "f16", True, "uniform"),
        (1, 2, 2, 1, 1, "f16", False, "standard"),
        (1, 2, 1, 129, 65, "bf16", False, "sharp"),
        (1, 2, 2, 3000, 9000, "f16", False, "sharp"),
    ],
)
def test_attention_target_matches_the_reference_contract(device, b, hq, hkv, sq, sk, dtype, causal, case):
    """Reference data case at N(0,1)*0.5, sampled rows of every head, online
    oracle with the policy's kv_tile, contract tolerance; plus the dense bar."""
    print(f"\n[fa] b={b} hq={hq} hkv={hkv} sq={sq} sk={sk} {dtype} causal={causal} case={case}", flush=True)
    data = inputs(b, hq, hkv, sq, sk, dtype, scale=0.5, case=case)
    actual = run_fa(data, dtype, causal, device)
    rows = sampled_rows(sq)
    expected = online_rows(data["q"], data["k"], data["v"], rows, dtype, causal, kv_tile(sq, sk))
    assert_contract(actual[:, :, rows], expected, dtype)
    if not causal:
        assert_baseline_bar(actual[:, :, rows], dense_reference(data["q"][:, :, rows], data["k"], data["v"], scale=128**-0.5))


@pytest.mark.parametrize("dtype,causal", [("f16", False), ("f16", True), ("bf16", False)])
def test_attention_target_full_output_matches_dense_fp32(device, dtype, causal):
    """Every row of a mid-sized problem against dense FP32 softmax (BASELINE bar)
    and the online oracle at the contract tolerance."""
    data = inputs(1, 4, 2, 512, 1536, dtype, scale=1.0)
    actual = run_fa(data, dtype, causal, device)
    ref = dense_reference(data["q"], data["k"], data["v"], scale=128**-0.5, causal=causal)
    assert_baseline_bar(actual, ref)
    rows = np.arange(512)
    assert_contract(actual, online_rows(data["q"], data["k"], data["v"], rows, dtype, causal, kv_tile(512, 1536)), dtype)


def test_uniform_keys_give_the_mean_of_values(device):
    data = inputs(1, 4, 2, 128, 1024, "bf16", case="uniform", scale=0.5)
    actual = run_fa(data, "bf16", False, device)
    for head in range(4):
        mean = rounded(data["v"][0, head // 2].mean(axis=0), "bf16")
        np.testing.assert_allclose(actual[0, head], np.broadcast_to(mean, (128, 128)), rtol=0.01, atol=0.001)


@pytest.mark.parametrize("dtype,causal", [("f16", False), ("f16", True), ("bf16", False)])
def test_flash_attention_c2_reference_sampled_rows(device, dtype, causal):
    """BASELINE configs[1] (B1 H32 D128 Sq = Sk = 8192, N(0,1) from the
    bench's seeded generator), non-causal and the causal row the bench also
    reports, in f16 and (non-causal) bf16: the reference's sampled scope, rows
    {0,7,63,64,71,127} of all 64 query tiles plus the last row, in every one
    of the 32 heads (benchmarks/validation/attention.py:91-104), against the
    online oracle with kv_tile 1024 at the contract tolerance of the dtype
    (contract.py:121-122)."""
    from ascendflow_amd.flash_attention import attention_target

    print(f"\n[fa] C2 B1 H32 S8192 {dtype} causal={causal}", flush=True)
    gen = torch.Generator(device=device)
    gen.manual_seed(9102201)
    shape = (1, 32, 8192, 128)
    q, k, v = (torch.randn(shape, generator=gen, device=device).to(TORCH[dtype]) for _ in range(3))
    o = torch.full_like(q, float("nan"))
    attention_target(q, k, v, o, 8192, 8192, B=1, HQ=32, HKV=32, D=128, DTYPE=dtype, SCALE=128**-0.5, CAUSAL=causal)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all(), "unwritten or non-finite output"
    rows = sampled_rows(8192)
    index = torch.as_tensor(rows, device=device)
    qs = q[0][:, index].float().cpu().numpy()
    ks, vs = k[0].float().cpu().numpy(), v[0].float().cpu().numpy()
    actual = o[0][:, index].float().cpu().numpy()
    block = kv_tile(8192, 8192)
    assert block == 1024
    for head in range(32):
        expected = np.concatenate([
            online_attention(qs[head, i : i + 128], ks[head], vs[head], block_kv=block, dtype=dtype,
                             scale=np.float32(1 / np.sqrt(128)), causal=causal, query_positions=rows[i : i + 128])
            for i in range(0, len(rows), 128)])
        assert_contract(actual[head], expected, dtype)


@pytest.mark.parametrize("case", ["random", "uniform"])
def test_simple_attention_matches_fp32(device, case):
    """H8, S1024, Sk128, D128 f16 (run_simple.py:83-84,115-118)."""
    from ascendflow_amd.flash_attention import simple_attention

    rng = np.random.default_rng(9102201)
    h, s = 8, 1024
    q = rounded(rng.standard_normal((h, s, 128)).astype(np.float32), "f16")
    k = rounded(rng.standard_normal((h, 128, 128)).astype(np.float32), "f16")
    v = rounded(rng.standard_normal((h, 128, 128)).astype(np.float32), "f16")
    if case == "uniform":
        k[:] = 0
    tq, tk, tv = (torch.from_numpy(x).to(device, torch.float16) for x in (q, k, v))
    o = torch.full_like(tq, float("nan"))
    simple_attention(tq, tk, tv, o, S=s, H=h)
    torch.cuda.synchronize()
    ref = simple_reference(q, k, v)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, rtol=0.002, atol=0.0005)
