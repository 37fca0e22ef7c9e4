"""GPU parity of the flash-attention and teaching-attention kernels against the CPU oracle."""

import numpy as np
import pytest
import torch

from oracle.attention import dense_reference, inputs, online_attention, simple_reference
from oracle.dtypes import rounded

pytestmark = pytest.mark.gpu

TORCH = {"f16": torch.float16, "bf16": torch.bfloat16}


def close_enough(actual, ref, dtype):
    """BASELINE bar max|err| <= 1e-2 * max|ref| plus an elementwise check at the
    reference contract's bf16 tolerance (benchmarks/attention/contract.py:121-122)."""
    err = float(np.max(np.abs(actual - ref)))
    bound = 1e-2 * float(np.max(np.abs(ref)))
    assert np.isfinite(actual).all()
    assert err <= bound, f"max|err| {err:.3g} > {bound:.3g}"
    np.testing.assert_allclose(actual, rounded(ref, dtype), rtol=0.01, atol=0.002)
    return err


def run_fa(data, dtype, causal, device, **kw):
    from ascendflow_amd.flash_attention import attention_target

    q, k, v = (torch.from_numpy(data[n]).to(device, TORCH[dtype]) for n in ("q", "k", "v"))
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    o = torch.full_like(q, float("nan"))
    attention_target(q, k, v, o, sq, sk, B=b, HQ=hq, HKV=hkv, D=d, DTYPE=dtype, SCALE=d**-0.5, CAUSAL=causal, **kw)
    torch.cuda.synchronize()
    return o.float().cpu().numpy()


@pytest.mark.parametrize(
    "b,hq,hkv,sq,sk,dtype,causal",
    [
        (1, 8, 8, 512, 512, "f16", False),
        (1, 8, 8, 512, 512, "f16", True),
        (2, 8, 2, 300, 700, "bf16", False),
        (2, 8, 2, 300, 700, "bf16", True),
        (1, 4, 1, 700, 300, "f16", True),
        (1, 2, 2, 1, 1, "f16", False),
        (1, 2, 1, 129, 65, "bf16", False),
    ],
)
def test_attention_target_matches_dense_fp32(device, b, hq, hkv, sq, sk, dtype, causal):
    print(f"\n[fa] b={b} hq={hq} hkv={hkv} sq={sq} sk={sk} {dtype} causal={causal}", flush=True)
    data = inputs(b, hq, hkv, sq, sk, dtype, scale=1.0)
    actual = run_fa(data, dtype, causal, device)
    ref = dense_reference(data["q"], data["k"], data["v"], scale=128**-0.5, causal=causal)
    close_enough(actual, ref, dtype)


def test_attention_target_matches_online_oracle_rows(device):
    """The restated reference recurrence (P rounded before PV, KV blocks of 1024)."""
    data = inputs(1, 2, 2, 256, 2048, "f16", scale=0.5)
    actual = run_fa(data, "f16", False, device)
    for head in range(2):
        ref = online_attention(data["q"][0, head], data["k"][0, head], data["v"][0, head], block_kv=1024, dtype="f16", scale=128**-0.5)
        np.testing.assert_allclose(actual[0, head], ref, rtol=0.01, atol=0.002)


def test_uniform_keys_give_the_mean_of_values(device):
    data = inputs(1, 4, 2, 128, 1024, "bf16", case="uniform", scale=0.5)
    actual = run_fa(data, "bf16", False, device)
    for head in range(4):
        mean = data["v"][0, head // 2].mean(axis=0)
        np.testing.assert_allclose(actual[0, head], np.broadcast_to(mean, (128, 128)), rtol=0.01, atol=0.002)


def test_flash_attention_c2_sampled_rows(device):
    """B1 H32 D128 Sq=Sk=8192 f16 non-causal, sampled query rows."""
    from ascendflow_amd.flash_attention import attention_target

    print("\n[fa] C2 B1 H32 S8192", flush=True)
    gen = torch.Generator(device=device)
    gen.manual_seed(9102201)
    shape = (1, 32, 8192, 128)
    q, k, v = (torch.randn(shape, generator=gen, device=device).to(torch.float16) for _ in range(3))
    o = torch.empty_like(q)
    attention_target(q, k, v, o, 8192, 8192, B=1, HQ=32, HKV=32, D=128, DTYPE="f16", SCALE=128**-0.5)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 127, 128, 4095, 4096, 8190, 8191])
    for head in (0, 17, 31):
        qh = q[0, head, rows].float().cpu().numpy()
        ref = dense_reference(qh[None, None], k[0, head].float().cpu().numpy()[None, None], v[0, head].float().cpu().numpy()[None, None], scale=128**-0.5)[0, 0]
        close_enough(o[0, head, rows].float().cpu().numpy(), ref, "f16")


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
