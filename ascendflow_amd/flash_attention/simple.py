"""Teaching attention with one resident 128-row KV tile, on MI355X.

Drop-in for ``examples/flash_attention/simple.py:60-69`` (``simple_attention``):
``softmax(Q K^T / sqrt(128)) V`` per head, FP16 Q/K/V/P/O with FP32 scores,
P normalised before its FP16 cast. Launches ``launch_simple_attention``.
"""

from __future__ import annotations

import torch

from .. import _native
from .._tensors import check_disjoint, check_tensor, require, stream_handle


def simple_attention(Q, K, V, O, S=256, H=4, GROUPS=20):
    require(S > 0 and S % 64 == 0, "S must be a positive multiple of 64")
    require(H > 0 and GROUPS > 0, "positive head and worker counts")
    check_tensor("Q", Q, (H, S, 128), torch.float16)
    check_tensor("K", K, (H, 128, 128), torch.float16, Q.device)
    check_tensor("V", V, (H, 128, 128), torch.float16, Q.device)
    check_tensor("O", O, (H, S, 128), torch.float16, Q.device)
    check_disjoint([("Q", Q, False), ("K", K, False), ("V", V, False), ("O", O, True)])
    status = _native.library().launch_simple_attention(
        stream_handle(Q.device), Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), None, S, H
    )
    _native.check(status, "launch_simple_attention")
    return O
