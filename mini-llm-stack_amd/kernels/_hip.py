"""Tensor plumbing shared by the kernel wrappers: dtype codes, device checks,
strides and the HIP stream of the calling thread."""

from __future__ import annotations

import torch

from kernels import MLS_BF16, MLS_F16, MLS_F32

_DT = {torch.float32: MLS_F32, torch.float16: MLS_F16, torch.bfloat16: MLS_BF16}


def dt_code(dtype: torch.dtype, what: str) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise TypeError(f"{what}: dtype {dtype} not supported (float32, float16, bfloat16)") from None


def require_hip(fn: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; the kernels have no host implementation."""
    dev = None
    for t in tensors:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{fn}: expected tensors, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise TypeError(f"{fn}: tensors must be on a HIP device (got {t.device}); "
                            "the gfx950 kernels have no CPU implementation")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{fn}: tensors on different devices ({dev} and {t.device})")
    return dev


def rows(t: torch.Tensor) -> torch.Tensor:
    """A 2-D view with unit inner stride (copying only if needed)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) < max(1, t.shape[1]):
        t = t.contiguous()
    return t


def ld(t: torch.Tensor) -> int:
    return max(int(t.stride(0)), int(t.shape[1]), 1)


def stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def scale_vector(scale: torch.Tensor) -> tuple[torch.Tensor, int]:
    """Per-row scales as fp32 or fp16 (kept as stored); other dtypes become fp32,
    which is what the reference does for every scale (dequant_matmul.py:147)."""
    if scale.dtype not in (torch.float32, torch.float16):
        scale = scale.to(torch.float32)
    return scale, _DT[scale.dtype]
