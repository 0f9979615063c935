"""INT8 straight-through-estimator linear on the gfx950 kernels: the INT8 part of
the reference's kernels/autograd_ops.py:95-134, under a module name of its own.

The reference's autograd_ops also holds the attention and MoE autograd functions
(autograd_ops.py:22-92), which this build does not replace. With the reference
checkout on sys.path after this package, the reference's autograd_ops imports
unchanged and its Int8MatmulSTE binds this package's int8_matmul / int8_dgrad;
this module serves callers without the checkout.

Forward: y = int8_matmul(x, W_q, s). Backward: dx = int8_dgrad(dy, W_q, s) on the
device, and the fp32 master weight receives dy^T @ x (a plain fp GEMM with nothing
quantized in it).
"""

from __future__ import annotations

import torch

from kernels.dequant_matmul import int8_dgrad, int8_matmul


class Int8MatmulSTE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w_q, scale, master_weight):
        ctx.save_for_backward(x, w_q, scale)
        return int8_matmul(x, w_q, scale)

    @staticmethod
    def backward(ctx, dy):
        x, w_q, scale = ctx.saved_tensors
        dy = dy.contiguous()
        dx = int8_dgrad(dy, w_q, scale)
        dw = dy.t() @ x
        return dx, None, None, dw


class QuantLinearSTE(torch.nn.Module):
    """Linear layer for quantization-aware training: the parameter stays fp32 and is
    re-quantized to INT8 (per-row scales) at every forward; its gradient passes straight
    through the quantizer."""

    def __init__(self, in_features: int, out_features: int):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.randn(out_features, in_features) * 0.02)

    def forward(self, x):
        from serve.quantize import quantize_int8
        w_q, scale = quantize_int8(self.weight.detach())
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        y = Int8MatmulSTE.apply(flat, w_q, scale, self.weight)
        return y.reshape(*shape[:-1], -1)
