"""Helpers shared by the sparse-MLA GPU tests: device copies of oracle inputs,
host views of device-built inputs, guard bytes and the tolerance contract."""

from __future__ import annotations

import numpy as np
import torch

from oracle import sparse_reference as sr
from oracle.dtypes import rounded

TORCH_DTYPE = {"bf16": torch.bfloat16, "f16": torch.float16}
INT_KEYS = ("cmp_sparse_indices", "ori_block_table", "cmp_block_table", "cu_seqlens_q", "seqused_ori_kv",
            "seqused_cmp_kv", "cmp_residual_kv", "ori_topk_length")
GUARD_WORDS = 256  # 512 guard bytes after the output (benchmarks/attention/run_sparse.py:31)


def to_device(data, policy, device):
    """Device tensors of an oracle input dict, plus a guarded output."""
    b16 = TORCH_DTYPE[policy["DTYPE"]]
    out = {name: torch.from_numpy(np.ascontiguousarray(data[name], np.float32)).to(device=device, dtype=b16)
           for name in ("q", "ori_kv", "cmp_kv")}
    for name in INT_KEYS:
        out[name] = torch.from_numpy(np.ascontiguousarray(data[name], np.int32)).to(device)
    out["sinks"] = torch.from_numpy(np.ascontiguousarray(data["sinks"], np.float32)).to(device)
    t, h, d = policy["T"], policy["H"], policy["D"]
    guarded = torch.full((t * h * d + GUARD_WORDS,), float("nan"), dtype=b16, device=device)
    out["_guarded"] = guarded
    out["attention_out"] = guarded[: t * h * d].view(t, h, d)
    return out


def call_args(tensors):
    return [tensors[name] for name in sr.TENSOR_ORDER]


def call_kwargs(policy):
    keys = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW", "TOPK", "S", "BM", "SCALE")
    return dict({k: policy[k] for k in keys}, DTYPE=policy["DTYPE"])


def guard_intact(tensors):
    tail = tensors["_guarded"][-GUARD_WORDS:]
    return bool(torch.isnan(tail.float()).all())


def host_view(inputs, tokens):
    """Oracle data dict for device-built ``SparseInputs``: metadata, patched caches,
    queries of ``tokens`` only (a dict keyed by token)."""
    policy, d = inputs.policy, inputs.policy["D"]
    data = {k: inputs.host[k] for k in INT_KEYS}
    data["sinks"] = inputs.tensors["sinks"].float().cpu().numpy()
    for name in ("ori_kv", "cmp_kv"):
        ids = inputs.touched[name]
        flat = inputs.tensors[name].view(-1, d)
        values = flat[torch.from_numpy(ids).to(flat.device)].float().cpu().numpy() if len(ids) else np.zeros((0, d), np.float32)
        data[name] = sr.PatchedRows(ids, values)
    index = torch.as_tensor(list(tokens), device=inputs.tensors["q"].device, dtype=torch.long)
    rows = inputs.tensors["q"][index].float().cpu().numpy()
    data["q"] = {token: rows[i] for i, token in enumerate(tokens)}
    return data


def expected_rows(data, policy, tokens):
    """Oracle selection as the kernel's debug image: int32 [n, S, 2]."""
    img = np.full((len(tokens), policy["S"], 2), -1, np.int32)
    for i, token in enumerate(tokens):
        for slot, cache, row in sr.selected_physical(data, policy, token):
            img[i, slot] = (cache, row)
    return img


def assert_close(actual, ref_fp32, dtype):
    """Tolerance contract: max|err| <= 1e-2 * max|ref| (BASELINE) and the
    reference runner's allclose(rtol=0.02, atol=0.005) (run_sparse.py:32)."""
    actual = np.asarray(actual, np.float32)
    ref = np.asarray(ref_fp32, np.float32)
    assert np.isfinite(actual).all(), "non-finite output"
    err = float(np.max(np.abs(actual - ref))) if ref.size else 0.0
    bound = 1e-2 * float(np.max(np.abs(ref))) if ref.size else 0.0
    assert err <= max(bound, 1e-6), f"max|err| {err:.3g} > 1e-2 * max|ref| = {bound:.3g}"
    np.testing.assert_allclose(actual, rounded(ref, dtype), rtol=0.02, atol=0.005)
    return err, bound
