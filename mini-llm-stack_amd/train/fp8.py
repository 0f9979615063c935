"""FP8 (e4m3) linear with per-tensor delayed scaling, on the gfx950 fp8 GEMM.

Same classes and behaviour as the reference's train/fp8.py (:33-131): the
forward quantizes x and W to e4m3 with delayed per-tensor scales and, when
use_kernel is set, multiplies them with kernels.fp8_matmul; otherwise it
multiplies the decoded operands in fp32. The backward re-quantizes dy to e5m2
(just-in-time scale) and computes both gradients against the same fp8 operands
the forward used. The reference always emulates the backward in fp32
(train/fp8.py:80-95); with use_kernel on a HIP device it runs here as two fp8
GEMMs with an e5m2 operand (dx = dy W: dy [M,N] e5m2 times W^T [K,N] e4m3;
dw = dy^T x: dy^T [N,M] times x^T [K,M]), the transposes materialised by a byte
transpose kernel; the exact datapath reproduces the emulation's fp32 result up
to summation order.
"""

from __future__ import annotations

from collections import deque

import torch
import torch.nn as nn

from kernels.fp8_matmul import (E4M3_MAX, E5M2_MAX, dequantize_e4m3, fp8_matmul, quantize_e4m3,
                                quantize_e4m3_t, quantize_e5m2, quantize_e5m2_t, transpose_u8)


class DynamicScaler:
    """One scale per tensor, chosen from the recent past: the largest |value| seen over
    the last `history` calls, divided by the format's largest finite value. The very
    first call has no past and uses the tensor's own maximum."""

    def __init__(self, fp8_max: float = E4M3_MAX, history: int = 16, enabled: bool = True):
        self.fp8_max = fp8_max
        self.hist: deque = deque(maxlen=history)
        self.enabled = enabled

    def scale_for(self, t: torch.Tensor) -> float:
        if not self.enabled:
            return 1.0
        amax = float(t.detach().abs().amax())
        if not self.hist:  # nothing recorded yet: seed the window with this tensor
            self.hist.append(max(amax, 1e-12))
        s = max(self.hist) / self.fp8_max
        self.hist.append(max(amax, 1e-12))
        return max(s, 1e-12)


def _quant_e5m2(x: torch.Tensor, scale: float) -> torch.Tensor:
    """train/fp8.py:50-52 (the HIP encoder on device tensors, bit-exact)."""
    return quantize_e5m2(x, scale)


def _dequant_e5m2(bits: torch.Tensor, scale: float) -> torch.Tensor:
    return bits.view(torch.float8_e5m2).float() * scale


class _FP8LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, sx, sw, use_kernel, scale_grads):
        ctx.scales = (sx, sw)
        ctx.scale_grads = scale_grads
        ctx.use_kernel = use_kernel
        ctx.transposed = False
        if use_kernel and x.device.type == "cuda" and any(ctx.needs_input_grad[:2]):
            # x and W encoded once into both layouts: the GEMM takes the row-major bytes,
            # the kernel backward needs only x^T and W^T, which are what is saved
            xb, xbt = quantize_e4m3_t(x, sx)
            wb, wbt = quantize_e4m3_t(w, sw)
            ctx.save_for_backward(xbt, wbt)
            ctx.transposed = True
            return fp8_matmul(xb, wb, sx, sw)
        xb = quantize_e4m3(x, sx)
        wb = quantize_e4m3(w, sw)
        ctx.save_for_backward(xb, wb)
        if use_kernel:
            return fp8_matmul(xb, wb, sx, sw)
        return dequantize_e4m3(xb, sx) @ dequantize_e4m3(wb, sw).t()

    @staticmethod
    def backward(ctx, dy):
        sx, sw = ctx.scales
        if ctx.scale_grads:
            sdy = max(float(dy.detach().abs().amax()) / E5M2_MAX, 1e-12)
        else:
            sdy = 1.0
        if ctx.use_kernel and dy.device.type == "cuda":
            if ctx.transposed:
                xbt, wbt = ctx.saved_tensors
            else:
                xb, wb = ctx.saved_tensors
                xbt, wbt = transpose_u8(xb), transpose_u8(wb)
            # the e5m2 gradient in both layouts from one pass (dy for dx, dy^T for dw)
            dyb, dybt = quantize_e5m2_t(dy, sdy)
            dx = fp8_matmul(dyb, wbt, sdy, sw, torch.float32, a_format="e5m2")
            dw = fp8_matmul(dybt, xbt, sdy, sx, torch.float32, a_format="e5m2")
            return dx, dw, None, None, None, None
        xb, wb = ctx.saved_tensors
        dyb = _quant_e5m2(dy, sdy)
        dyh = _dequant_e5m2(dyb, sdy)
        xh = dequantize_e4m3(xb, sx)
        wh = dequantize_e4m3(wb, sw)
        return dyh @ wh, dyh.t() @ xh, None, None, None, None


class FP8Linear(nn.Module):
    def __init__(self, linear: nn.Linear, enabled: bool = True, use_kernel: bool = False):
        super().__init__()
        self.weight = nn.Parameter(linear.weight.detach().clone())
        self.sx = DynamicScaler(enabled=enabled)
        self.sw = DynamicScaler(enabled=enabled)
        self.use_kernel = use_kernel

    def forward(self, x):
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        y = _FP8LinearFn.apply(flat, self.weight, self.sx.scale_for(flat),
                               self.sw.scale_for(self.weight), self.use_kernel,
                               self.sx.enabled)
        return y.reshape(*shape[:-1], -1)


def convert_linears_to_fp8(model: nn.Module, enabled: bool = True,
                           use_kernel: bool = False) -> nn.Module:
    """Swap every attention (wq/wk/wv/wo) and MLP (w_gate/w_up/w_down) linear for
    FP8Linear; embeddings, head and norms stay fp32 (train/fp8.py:117-131). Modules
    are recognised by their slot names rather than by class."""
    import copy
    model = copy.deepcopy(model)
    for m in model.modules():
        for names in (("wq", "wk", "wv", "wo"), ("w_gate", "w_up", "w_down")):
            if all(isinstance(getattr(m, n, None), nn.Linear) for n in names):
                for n in names:
                    setattr(m, n, FP8Linear(getattr(m, n), enabled, use_kernel))
    return model
