"""b16 storage codec for the oracle (test infrastructure only).

Restates ``benchmarks/validation/dtypes.py:6-26``: FP32 -> bf16 rounds to
nearest, ties to even, by adding ``0x7FFF + lsb`` to the FP32 bit pattern and
keeping the upper half; f16 uses IEEE conversion (NumPy ``astype``).
Pinned by ``tests/test_oracle_dtypes.py`` (the reference's ties-to-even vectors
``tests/operators/test_attention_math.py:14-19`` plus a brute-force comparison
with torch's bf16 conversion over many random and edge-case values).
"""

from __future__ import annotations

import numpy as np

B16 = ("bf16", "f16")


def _check(dtype: str) -> None:
    if dtype not in B16:
        raise ValueError(f"oracle needs an explicit b16 dtype, got {dtype!r}")


def encode(values, dtype: str) -> np.ndarray:
    """FP32 values -> uint16 storage words (same shape)."""
    _check(dtype)
    values = np.ascontiguousarray(values, dtype=np.float32)
    if dtype == "f16":
        return values.astype(np.float16).view(np.uint16)
    bits = values.view(np.uint32).astype(np.uint64)
    lsb = (bits >> np.uint64(16)) & np.uint64(1)
    upper = (bits + np.uint64(0x7FFF) + lsb) >> np.uint64(16)
    return (upper & np.uint64(0xFFFF)).astype(np.uint16)


def decode(words, dtype: str) -> np.ndarray:
    """uint16 storage words -> FP32 values (same shape)."""
    _check(dtype)
    words = np.ascontiguousarray(words, dtype=np.uint16)
    if dtype == "f16":
        return words.view(np.float16).astype(np.float32)
    return (words.astype(np.uint32) << np.uint32(16)).view(np.float32)


def rounded(values, dtype: str) -> np.ndarray:
    """Round FP32 values through b16 storage and back."""
    return decode(encode(values, dtype), dtype)
