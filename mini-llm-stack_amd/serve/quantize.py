"""Weight-only quantization: INT8 (per-row symmetric) and INT4 (group-wise).

Same functions, classes and buffer layouts as the reference's serve/quantize.py
(:18-129), so a serving engine built on nn.Linear slots runs unchanged:

INT8: scale[n] = max|w[n]| / 127 (floored at 1e-8); w_q = round-half-even(w / scale)
      clamped to [-127, 127].
INT4: per group of `group_size` along K, scale = max|w_group| / 7 (floored at
      1e-8); q = clamp(round(w / scale), -8, 7) + 8, two nibbles per byte with
      even k in the low nibble.

Quantization is load-time work. On HIP tensors it runs the gfx950 quantizer
kernels (bit-exact: IEEE division, ties to even); on host tensors (a model
quantized before it is moved to the GPU, as the reference's CLI does) it runs
the reference's host op sequence, which is the definition the kernels match.
QuantLinear(use_kernel=True) runs the fused HIP GEMMs of kernels.dequant_matmul;
use_kernel=False keeps the reference's dequantize-then-matmul path.

Unlike the reference, this module does not import the model package (the
reference imports train.model only for a type annotation, :15): quantize_model
finds the Linear slots by attribute name.
"""

from __future__ import annotations

import torch
import torch.nn as nn


def _hip_quantizer():
    import kernels
    from kernels._hip import ld, stream
    return kernels, ld, stream


def quantize_int8(w: torch.Tensor):
    """(w_q int8 [N, K], scale fp32 [N]) -- serve/quantize.py:18-21."""
    if w.device.type != "cuda":
        scale = (w.abs().amax(dim=1) / 127.0).clamp(min=1e-8)
        w_q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
        return w_q, scale
    kernels, ld, stream = _hip_quantizer()
    w32 = w.detach().to(torch.float32)
    if w32.stride(1) != 1:
        w32 = w32.contiguous()
    N, K = w32.shape
    w_q = torch.empty(N, K, dtype=torch.int8, device=w.device)
    scale = torch.empty(N, dtype=torch.float32, device=w.device)
    kernels.check(kernels.lib().mls_quantize_int8(
        w32.data_ptr(), N, K, ld(w32), w_q.data_ptr(), ld(w_q), scale.data_ptr(),
        stream(w.device)), "quantize_int8")
    return w_q, scale


def dequantize_int8(w_q: torch.Tensor, scale: torch.Tensor):
    return w_q.float() * scale[:, None]


def quantize_int4(w: torch.Tensor, group_size: int = 32):
    """(packed uint8 [N, K/2], scale fp32 [N, K/group_size]) -- serve/quantize.py:28-36."""
    N, K = w.shape
    assert K % group_size == 0
    if w.device.type != "cuda" or group_size % 2 or K % 2:
        g = w.reshape(N, K // group_size, group_size)
        scale = (g.abs().amax(dim=2) / 7.0).clamp(min=1e-8)
        q = torch.round(g / scale[:, :, None]).clamp(-8, 7) + 8
        q = q.reshape(N, K).to(torch.uint8)
        packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
        return packed, scale
    kernels, ld, stream = _hip_quantizer()
    w32 = w.detach().to(torch.float32)
    if w32.stride(1) != 1:
        w32 = w32.contiguous()
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=w.device)
    scale = torch.empty(N, K // group_size, dtype=torch.float32, device=w.device)
    kernels.check(kernels.lib().mls_quantize_int4(
        w32.data_ptr(), N, K, ld(w32), group_size, packed.data_ptr(), ld(packed),
        scale.data_ptr(), stream(w.device)), "quantize_int4")
    return packed, scale


def dequantize_int4(packed: torch.Tensor, scale: torch.Tensor, group_size: int):
    N = packed.shape[0]
    K = packed.shape[1] * 2
    q = torch.empty(N, K, dtype=torch.uint8, device=packed.device)
    q[:, 0::2] = packed & 0x0F
    q[:, 1::2] = packed >> 4
    w = q.float() - 8.0
    w = w.reshape(N, K // group_size, group_size) * scale.float()[:, :, None]
    return w.reshape(N, K)


class QuantLinear(nn.Module):
    """Drop-in nn.Linear replacement holding quantized weights (serve/quantize.py:50-95).

    use_kernel=True runs the fused gfx950 dequant GEMM; False runs the
    reference path (explicit dequant then matmul), kept for correctness tests
    and host execution.
    """

    def __init__(self, linear: nn.Linear, bits: int = 8, group_size: int = 32,
                 use_kernel: bool = True):
        super().__init__()
        assert linear.bias is None
        assert bits in (4, 8)
        self.bits, self.group_size, self.use_kernel = bits, group_size, use_kernel
        self.out_features, self.in_features = linear.weight.shape
        w = linear.weight.detach().float()
        if bits == 8:
            w_q, scale = quantize_int8(w)
        else:
            w_q, scale = quantize_int4(w, group_size)
        self.register_buffer("w_q", w_q)
        self.register_buffer("scale", scale)

    def dequant(self) -> torch.Tensor:
        if self.bits == 8:
            return dequantize_int8(self.w_q, self.scale)
        return dequantize_int4(self.w_q, self.scale, self.group_size)

    def weight_bytes(self) -> int:
        return self.w_q.numel() * self.w_q.element_size() + \
            self.scale.numel() * self.scale.element_size()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.reshape(-1, self.in_features)
        if self.use_kernel:
            from kernels.dequant_matmul import int4_matmul, int8_matmul
            if self.bits == 8:
                y = int8_matmul(flat, self.w_q, self.scale)
            else:
                y = int4_matmul(flat, self.w_q, self.scale, self.group_size)
        else:
            y = flat @ self.dequant().to(flat.dtype).t()
        return y.reshape(*shape[:-1], self.out_features)


_ATTN_SLOTS = ("wq", "wk", "wv", "wo")
_MLP_SLOTS = ("w_gate", "w_up", "w_down")


def quantize_model(model: nn.Module, bits: int = 8, group_size: int = 32,
                   use_kernel: bool = True) -> nn.Module:
    """Replace all block linears with QuantLinear (router/embed/head stay fp)
    (serve/quantize.py:98-115). Walks model.blocks; each block's .attn holds
    wq/wk/wv/wo and its .mlp holds w_gate/w_up/w_down, or, when blk.is_moe,
    .mlp.experts is a list of such MLPs."""
    import copy
    model = copy.deepcopy(model)
    for blk in model.blocks:
        a = blk.attn
        for name in _ATTN_SLOTS:
            setattr(a, name, QuantLinear(getattr(a, name), bits, group_size, use_kernel))
        mods = blk.mlp.experts if getattr(blk, "is_moe", False) else [blk.mlp]
        for m in mods:
            for name in _MLP_SLOTS:
                setattr(m, name, QuantLinear(getattr(m, name), bits, group_size, use_kernel))
    return model


def model_weight_bytes(model: nn.Module) -> int:
    """Bytes of QuantLinear buffers plus every distinct parameter (serve/quantize.py:118-129)."""
    total = 0
    seen = set()
    for m in model.modules():
        if isinstance(m, QuantLinear):
            total += m.weight_bytes()
    for p in model.parameters():
        if id(p) in seen:
            continue
        seen.add(id(p))
        total += p.numel() * p.element_size()
    return total
