"""Tensor-argument checks shared by the operator entries.

Mirrors the checks the reference's TensorKernel applies before a launch
(src/runtime/torch.py:94-167): shape, dtype, device, contiguity and pairwise
disjointness of the external tensors. Launchers themselves never read tensor
values, as in the reference (docs/operators/sparse-mla.md:83-84).
"""

from __future__ import annotations

import torch

DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}


def storage_dtype(value) -> str:
    """Normalise a DTYPE constexpr ("bf16"/"f16", torch dtype or an object named so)."""
    if isinstance(value, torch.dtype):
        for name, dt in DTYPES.items():
            if dt == value:
                return name
    name = str(getattr(value, "name", value)).lower().replace("torch.", "")
    aliases = {"bfloat16": "bf16", "float16": "f16", "half": "f16", "bf16": "bf16", "f16": "f16"}
    if name not in aliases:
        raise ValueError(f"unsupported storage dtype {value!r}; expected bf16 or f16")
    return aliases[name]


def require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def check_tensor(name, tensor, shape, dtype, device=None):
    require(isinstance(tensor, torch.Tensor), f"{name} must be a torch.Tensor")
    require(tuple(tensor.shape) == tuple(shape), f"{name} shape {tuple(tensor.shape)} != {tuple(shape)}")
    require(tensor.dtype == dtype, f"{name} dtype {tensor.dtype} != {dtype}")
    require(tensor.is_cuda, f"{name} must live on a ROCm device")
    require(tensor.is_contiguous(), f"{name} must be contiguous")
    if device is not None:
        require(tensor.device == device, f"{name} is on {tensor.device}, expected {device}")


def _span(tensor):
    start = tensor.data_ptr()
    return start, start + tensor.numel() * tensor.element_size()


def check_disjoint(named):
    """Every written tensor must not overlap any other external tensor (read
    tensors may share memory with each other, as read-only caches do)."""
    spans = [(name, *_span(t), write) for name, t, write in named if t.numel()]
    for i, (a, a0, a1, aw) in enumerate(spans):
        if not aw:
            continue
        for j, (b, b0, b1, _) in enumerate(spans):
            if j != i and a0 < b1 and b0 < a1:
                first, second = (a, b) if i < j else (b, a)
                raise ValueError(f"external tensors {first} and {second} overlap")


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
