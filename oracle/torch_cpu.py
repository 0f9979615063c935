"""The reference's PyTorch CPU path for this layer — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

bench.py's cpu_baseline leg times these functions on the GPU box's host cores: they
are the reference's own torch op sequences for a quantized linear when no kernel
runs (QuantLinear(use_kernel=False)) and for the FP8 linear's emulation path,
restated here so that nothing from the reference travels to the box. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this file.

Pins (tests/test_oracle.py): the dequantizers equal oracle.ref's numpy ones
bit for bit (and so the golden quantizer fixtures); the linears equal oracle.ref's
GEMMs within the fp32 bound (same products, different summation order).
"""

from __future__ import annotations

import torch


def dequantize_int8(w_q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """serve/quantize.py:24-25."""
    return w_q.float() * scale[:, None]


def dequantize_int4(packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """serve/quantize.py:39-47: unpack (even k from the low nibble), minus 8, times the
    group scale, in fp32."""
    N = packed.shape[0]
    K = packed.shape[1] * 2
    q = torch.empty(N, K, dtype=torch.uint8, device=packed.device)
    q[:, 0::2] = packed & 0x0F
    q[:, 1::2] = packed >> 4
    w = q.float() - 8.0
    return (w.reshape(N, K // group_size, group_size) * scale[:, :, None]).reshape(N, K)


def quant_linear(x: torch.Tensor, w_q: torch.Tensor, scale: torch.Tensor, bits: int,
                 group_size: int = 0) -> torch.Tensor:
    """QuantLinear.forward with use_kernel=False (serve/quantize.py:75-78, 84-95): the
    weights dequantized to fp32, rounded to x's dtype, then x @ W^T in x's dtype."""
    flat = x.reshape(-1, x.shape[-1])
    w = dequantize_int8(w_q, scale) if bits == 8 else dequantize_int4(w_q, scale, group_size)
    y = flat @ w.to(flat.dtype).t()
    return y.reshape(*x.shape[:-1], w.shape[0])


def dequantize_e4m3(bits: torch.Tensor, scale) -> torch.Tensor:
    """kernels/fp8_matmul.py:109-110; a [rows, 1] scale tensor broadcasts per row."""
    return bits.view(torch.float8_e4m3fn).float() * scale


def fp8_linear_emulated(a_bits: torch.Tensor, b_bits: torch.Tensor, sa, sb) -> torch.Tensor:
    """The FP8 linear's emulation path (train/fp8.py:76-77): both e4m3 operands
    decoded and scaled in fp32, then an fp32 matmul."""
    return dequantize_e4m3(a_bits, sa) @ dequantize_e4m3(b_bits, sb).t()
