"""OCP e4m3 ("fn") codec and the e4m3 GEMM with inline scales.

Same names and call signatures as the reference (kernels/fp8_matmul.py:34-128).
e4m3fn: 1 sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities,
NaN = S.1111.111, max finite 448.

fp8_matmul has two gfx950 datapaths. The default widens both e4m3 operands to
bf16 (exact) while staging them into LDS and multiplies on the bf16 matrix cores,
whose fp32 accumulation reproduces the reference's decode-then-fp32-dot result
(kernels/fp8_matmul.py:50-81). native=True (or MLS_FP8_NATIVE=1 in the
environment) feeds the raw bytes to the fp8 matrix cores
(v_mfma_f32_16x16x128_f8f6f4) at twice the peak rate; that instruction truncates
each product of a group of 8 toward zero at 2^-13 of the group's largest before
adding them, so rows with outliers deviate from the fp32 result by up to ~2^-13 of
the largest product per product of the group. Scales are applied in the epilogue and may be Python floats
(per tensor, the reference's form), 0-d tensors, or fp32 tensors of shape [M] /
[N] (per row).

fp8_matmul(..., a_format="e5m2") takes an e5m2 A operand (FP8 training's gradients;
e5m2 widens to bf16 exactly, and the native path selects the MFMA's bf8 format);
quantize_e5m2, transpose_u8 and the encoders with a transposed copy (quantize_e5m2_t,
quantize_e4m3_t) are the other pieces of that backward.

quantize_e4m3 / dequantize_e4m3 run the gfx950 codec kernels on HIP tensors. On
host tensors (the load-time and CPU-training callers) they run the reference's
own host op sequence, which is the definition the HIP codec is bit-exact to.
"""

from __future__ import annotations

import os

import torch

import kernels
from kernels._hip import dt_code, ld, require_hip, rows, stream

E4M3_MAX = 448.0
E5M2_MAX = 57344.0
_FORMATS = {"e4m3": 0, "e5m2": kernels.MLS_FP8_A_E5M2}


def decode_e4m3(bits: torch.Tensor) -> torch.Tensor:
    """Kernel-decode a uint8 tensor of e4m3fn bit patterns to fp32; the NaN
    patterns 0x7F / 0xFF decode to 0 (kernels/fp8_matmul.py:37-47, 93-100)."""
    dev = require_hip("decode_e4m3", bits)
    if bits.dtype not in (torch.uint8, torch.float8_e4m3fn):
        raise TypeError(f"decode_e4m3: expected uint8 bits, got {bits.dtype}")
    flat = bits.reshape(-1).contiguous().view(torch.uint8)
    out = torch.empty(flat.shape, dtype=torch.float32, device=dev)
    kernels.check(kernels.lib().mls_e4m3_decode(flat.data_ptr(), out.data_ptr(), flat.numel(),
                                                stream(dev)), "decode_e4m3")
    return out.reshape(bits.shape)


def _row_scale(scale, rows_: int, dev, what: str, per_row_1d: bool):
    """(scalar, pointer, stride, keepalive) for a scale that is per tensor (a float
    or a 1-element tensor) or per row of a [rows_, cols] operand (shape [rows_, 1],
    or [rows_] when per_row_1d). None when the scale needs general broadcasting."""
    if not isinstance(scale, torch.Tensor):
        return float(scale), None, 0, None
    if scale.device != dev:
        raise ValueError(f"{what}: scale on {scale.device}, operand on {dev}")
    s = scale.to(torch.float32)
    if s.numel() == 1:
        s = s.reshape(1)
        return 0.0, s.data_ptr(), 0, s
    per_row = (s.dim() == 2 and tuple(s.shape) == (rows_, 1)) or \
        (per_row_1d and s.dim() == 1 and s.shape[0] == rows_)
    if per_row:
        s = s.reshape(-1).contiguous()
        return 0.0, s.data_ptr(), 1, s
    return None


def quantize_e4m3(x: torch.Tensor, scale) -> torch.Tensor:
    """e4m3 bits of x / scale, saturated to ±448, round to nearest even
    (kernels/fp8_matmul.py:103-106). Returns uint8. `scale` broadcasts as in
    torch: a float, a 1-element tensor, [M, 1] per row of a 2-D x, or any other
    broadcastable tensor."""
    if x.device.type != "cuda":
        q = (x.float() / scale).clamp(-E4M3_MAX, E4M3_MAX)
        return q.to(torch.float8_e4m3fn).view(torch.uint8)
    dev = x.device
    shape = x.shape
    xdt = dt_code(x.dtype, "quantize_e4m3")
    x2 = rows(x.reshape(1, 1) if x.dim() == 0 else x.reshape(-1, shape[-1]))
    sa = _row_scale(scale, x2.shape[0], dev, "quantize_e4m3", False) \
        if x.dim() <= 2 or not isinstance(scale, torch.Tensor) or scale.numel() == 1 else None
    if sa is None:
        # general broadcast: IEEE division on the device (tensor / tensor is a true
        # division in torch), then encode with scale 1 (division by 1 is exact)
        q = x.float() / scale
        shape = q.shape
        x2 = rows(q.reshape(1, 1) if q.dim() == 0 else q.reshape(-1, shape[-1]))
        xdt, sa = dt_code(torch.float32, "quantize_e4m3"), (1.0, None, 0, None)
    out = torch.empty(x2.shape, dtype=torch.uint8, device=dev)
    kernels.check(kernels.lib().mls_e4m3_encode(
        x2.data_ptr(), xdt, x2.shape[0], x2.shape[1], ld(x2), sa[0], sa[1], sa[2],
        out.data_ptr(), ld(out), stream(dev)), "quantize_e4m3")
    return out.reshape(shape)


def quantize_e5m2(x: torch.Tensor, scale) -> torch.Tensor:
    """e5m2 bits of x / scale, clamped to ±57344, round to nearest even: the
    gradient quantizer of FP8 training (train/fp8.py:50-52). Returns uint8. scale: a
    float, a 1-element tensor or [M, 1] per row of a 2-D x."""
    if x.device.type != "cuda":
        q = (x.float() / scale).clamp(-E5M2_MAX, E5M2_MAX)
        return q.to(torch.float8_e5m2).view(torch.uint8)
    dev = x.device
    shape = x.shape
    x2 = rows(x.reshape(1, 1) if x.dim() == 0 else x.reshape(-1, shape[-1]))
    sa = _row_scale(scale, x2.shape[0], dev, "quantize_e5m2", False) \
        if x.dim() <= 2 or not isinstance(scale, torch.Tensor) or scale.numel() == 1 else None
    if sa is None:
        raise ValueError("quantize_e5m2: scale must be a float, a 1-element tensor or [M, 1]")
    out = torch.empty(x2.shape, dtype=torch.uint8, device=dev)
    kernels.check(kernels.lib().mls_e5m2_encode(
        x2.data_ptr(), dt_code(x.dtype, "quantize_e5m2"), x2.shape[0], x2.shape[1], ld(x2), sa[0], sa[1], sa[2],
        out.data_ptr(), ld(out), stream(dev)), "quantize_e5m2")
    return out.reshape(shape)


def _encode_t(fn: str, entry: str, x: torch.Tensor, scale) -> tuple[torch.Tensor, torch.Tensor]:
    dev = require_hip(fn, x)
    if x.dim() != 2:
        raise ValueError(f"{fn}: expected a 2-D tensor, got {tuple(x.shape)}")
    x2 = rows(x)
    R, C = x2.shape
    sa = _row_scale(scale, R, dev, fn, False)
    if sa is None:
        raise ValueError(f"{fn}: scale must be a float, a 1-element tensor or [M, 1]")
    out = torch.empty(R, C, dtype=torch.uint8, device=dev)
    out_t = torch.empty(C, R, dtype=torch.uint8, device=dev)
    kernels.check(getattr(kernels.lib(), entry)(
        x2.data_ptr(), dt_code(x.dtype, fn), R, C, ld(x2), sa[0], sa[1], sa[2],
        out.data_ptr(), ld(out), out_t.data_ptr(), ld(out_t), stream(dev)), fn)
    return out, out_t


def quantize_e5m2_t(x: torch.Tensor, scale) -> tuple[torch.Tensor, torch.Tensor]:
    """(quantize_e5m2(x, scale), its transpose as a contiguous [cols, rows] uint8 tensor)
    from one pass over a 2-D device tensor x: the gradient operand of FP8 training's
    backward in both layouts it needs (train/fp8.py:88-94). scale: a float, a 1-element
    tensor or [M, 1] per row."""
    return _encode_t("quantize_e5m2_t", "mls_e5m2_encode_t", x, scale)


def quantize_e4m3_t(x: torch.Tensor, scale) -> tuple[torch.Tensor, torch.Tensor]:
    """(quantize_e4m3(x, scale), its transpose as a contiguous [cols, rows] uint8 tensor)
    from one pass over a 2-D device tensor x: FP8Linear's forward operands, whose
    transposes its backward needs (train/fp8.py:68-69, 88-94). scale: a float, a
    1-element tensor or [M, 1] per row."""
    return _encode_t("quantize_e4m3_t", "mls_e4m3_encode_t", x, scale)


def transpose_u8(t: torch.Tensor) -> torch.Tensor:
    """A contiguous [cols, rows] copy of a 2-D byte tensor (fp8 bits): the .t() of
    an fp8 operand, materialised for the K-contiguous GEMM."""
    dev = require_hip("transpose_u8", t)
    if t.dim() != 2 or t.element_size() != 1:
        raise ValueError(f"transpose_u8: expected a 2-D byte tensor, got {t.dtype} {tuple(t.shape)}")
    src = rows(t.view(torch.uint8))
    R, C = src.shape
    out = torch.empty(C, R, dtype=torch.uint8, device=dev)
    kernels.check(kernels.lib().mls_transpose_u8(src.data_ptr(), R, C, ld(src), out.data_ptr(), ld(out),
                                                 stream(dev)), "transpose_u8")
    return out


def dequantize_e4m3(bits: torch.Tensor, scale) -> torch.Tensor:
    """value(bits) * scale in fp32; the NaN patterns stay NaN, as in torch's float8
    view (kernels/fp8_matmul.py:109-110)."""
    if bits.device.type != "cuda":
        return bits.view(torch.float8_e4m3fn).float() * scale
    dev = bits.device
    shape = bits.shape
    u8 = bits.view(torch.uint8)
    b2 = rows(u8.reshape(1, 1) if u8.dim() == 0 else u8.reshape(-1, shape[-1]))
    sa = _row_scale(scale, b2.shape[0], dev, "dequantize_e4m3", False) \
        if bits.dim() <= 2 or not isinstance(scale, torch.Tensor) or scale.numel() == 1 else None
    if sa is None:  # general broadcast: exact decode, then one fp32 multiply on the device
        return dequantize_e4m3(bits, 1.0) * scale
    out = torch.empty(b2.shape, dtype=torch.float32, device=dev)
    kernels.check(kernels.lib().mls_e4m3_dequantize(
        b2.data_ptr(), b2.shape[0], b2.shape[1], ld(b2), sa[0], sa[1], sa[2],
        out.data_ptr(), ld(out), stream(dev)), "dequantize_e4m3")
    return out.reshape(shape)


def fp8_matmul(a_bits: torch.Tensor, b_bits: torch.Tensor,
               sa, sb, out_dtype: torch.dtype = torch.float32, *,
               native: bool | None = None, a_format: str = "e4m3") -> torch.Tensor:
    """a_bits [M,K], b_bits [N,K] uint8 e4m3 -> sa*sb*(Â @ B̂ᵀ) [M,N]
    (kernels/fp8_matmul.py:113-128). sa / sb: float, 0-d tensor, or fp32 [M] / [N].
    native: use the fp8 matrix cores (see the module docstring); default from
    MLS_FP8_NATIVE, else the exact bf16 datapath. a_format="e5m2": a_bits holds
    e5m2 bytes (the gradient operand of FP8 training's backward, train/fp8.py:80-95)."""
    if a_format not in _FORMATS:
        raise ValueError(f"fp8_matmul: a_format {a_format!r} (e4m3 or e5m2)")
    if native is None:
        native = os.environ.get("MLS_FP8_NATIVE", "0") not in ("", "0")
    dev = require_hip("fp8_matmul", a_bits, b_bits)
    M, K = a_bits.shape
    N = b_bits.shape[0]
    if b_bits.shape[1] != K:
        raise ValueError(f"fp8_matmul: K mismatch {tuple(a_bits.shape)} vs {tuple(b_bits.shape)}")
    cdt = dt_code(out_dtype, "fp8_matmul out_dtype")
    a2, b2 = rows(a_bits.view(torch.uint8)), rows(b_bits.view(torch.uint8))
    sa_args = _row_scale(sa, M, dev, "fp8_matmul sa", True)
    sb_args = _row_scale(sb, N, dev, "fp8_matmul sb", True)
    if sa_args is None or sb_args is None:
        raise ValueError("fp8_matmul: scales must be floats, 0-d tensors or per-row [M] / [N]")
    c = torch.empty(M, N, dtype=out_dtype, device=dev)
    kernels.check(kernels.lib().mls_fp8_gemm(
        a2.data_ptr(), ld(a2), b2.data_ptr(), ld(b2),
        sa_args[0], sa_args[1], sa_args[2], sb_args[0], sb_args[1], sb_args[2],
        c.data_ptr(), cdt, ld(c), M, N, K, (kernels.MLS_FP8_NATIVE if native else 0) | _FORMATS[a_format],
        stream(dev)),
        "fp8_matmul")
    return c
