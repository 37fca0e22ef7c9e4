"""BNSD flash attention forward on MI355X.

Drop-in for ``examples/flash_attention/attention.py:243-264`` (``attention_target``)
and its host tiling policy ``causal_policy`` (``attention.py:19-26``). The call
launches the fused gfx950 kernel of ``csrc/flash_attention.hip`` through
``launch_attention_target`` on the current stream. The Ascend tiling
constexprs (BQ, BM, BK, CK, VR, GROUPS) are checked against the reference's
asserts (``attention.py:305-318``) and otherwise ignored.
"""

from __future__ import annotations

import ctypes as ct

from .. import _native
from .._tensors import DTYPES, check_disjoint, check_tensor, require, storage_dtype, stream_handle


def causal_policy(sq, sk):
    """Host tiling policy of the reference (``attention.py:19-26``), unchanged."""
    prefix = min(sq, sk)
    if prefix < 2048:
        return {"kv_tile": 256, "vector_rows": 16}
    if prefix < 8192:
        return {"kv_tile": 512, "vector_rows": 16}
    return {"kv_tile": 1024, "vector_rows": 8}


def attention_target(
    Q,
    K,
    V,
    O,
    Sq,
    Sk,
    B=1,
    HQ=8,
    HKV=8,
    D=128,
    BQ=256,
    BM=128,
    BK=1024,
    CK=128,
    VR=8,
    GROUPS=20,
    DTYPE="f16",
    SCALE=0.08838834764831845,
    CAUSAL=False,
):
    """FA forward: O[B,HQ,Sq,D] = softmax(Q K^T * SCALE [+ causal mask]) V."""
    dtype = storage_dtype(DTYPE)
    Sq, Sk = int(Sq), int(Sk)
    require(Sq >= 1 and Sk >= 1, "Sq and Sk must be >= 1")
    require(B > 0 and HQ > 0 and HKV > 0, "positive batch and head counts")
    require(HQ % HKV == 0, "query heads must be divisible by KV heads")
    require(VR > 0 and BQ % (2 * VR) == 0, "query tile must cover complete rows on both AIVs")
    require(BM > 0 and BQ % BM == 0 and BQ <= 2 * BM, "query tile must fit the accumulator planes")
    require(CK > 0 and BK % CK == 0 and CK == D, "KV tile must contain complete CK == D chunks")
    require(GROUPS > 0 and SCALE > 0, "positive worker count and scale")
    require(D == 128, "gfx950 kernel supports D = 128")
    b16 = DTYPES[dtype]
    check_tensor("Q", Q, (B, HQ, Sq, D), b16)
    check_tensor("K", K, (B, HKV, Sk, D), b16, Q.device)
    check_tensor("V", V, (B, HKV, Sk, D), b16, Q.device)
    check_tensor("O", O, (B, HQ, Sq, D), b16, Q.device)
    check_disjoint([("Q", Q, False), ("K", K, False), ("V", V, False), ("O", O, True)])
    params = _native.FaParams(
        B=B, HQ=HQ, HKV=HKV, D=D, dtype=_native.AFA_DTYPE[dtype], causal=int(bool(CAUSAL)), scale=SCALE, reserved=0
    )
    status = _native.library().launch_attention_target(
        stream_handle(Q.device), Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), None, Sq, Sk, ct.byref(params)
    )
    _native.check(status, "launch_attention_target")
    return O
