"""Weight-only INT8 / INT4 GEMMs with the dequantization inside the kernel.

Same call signatures and layouts as the reference module
(kernels/dequant_matmul.py:17-25, 140-185):

INT8: w_q [N, K] int8 with one symmetric scale per output row, s[N];
      y = (a @ w_q^T) * s, the scale applied once after fp32 accumulation.
INT4: w_packed [N, K/2] uint8, two nibbles per byte (even k in the low nibble),
      stored value = q + 8, group scales s[N, K/group]; y = a @ ((v - 8) * s)^T.

The work runs in libmls_hip.so on gfx950 (include/mls.h): a decode GEMV that
streams the packed weights with 16-byte loads for small M, and an MFMA GEMM that
dequantizes weight tiles into LDS for larger M. The library picks the kernel
from the shape. fp32 activations with M >= 2 (the reference's fp32 engine) run on
the bf16 matrix cores as hi + lo parts, x split into a workspace taken from torch's
caching allocator. Outputs have a.dtype; scales may be fp32 or fp16 (other float
dtypes are converted to fp32, as the reference does for every scale).
"""

from __future__ import annotations

import torch

import kernels
from kernels._hip import dt_code, ld, require_hip, rows, scale_vector, stream


def int8_matmul(a: torch.Tensor, w_q: torch.Tensor, scale: torch.Tensor):
    """a [M, K] fp  @  dequant(w_q [N, K] int8, scale [N]).T  ->  [M, N]
    (kernels/dequant_matmul.py:140-152)."""
    dev = require_hip("int8_matmul", a, w_q, scale)
    M, K = a.shape
    N = w_q.shape[0]
    if w_q.dtype != torch.int8:
        raise TypeError(f"int8_matmul: w_q must be int8, got {w_q.dtype}")
    if w_q.dim() != 2 or w_q.shape[1] != K:
        raise ValueError(f"int8_matmul: w_q shape {tuple(w_q.shape)} does not match K={K}")
    if scale.numel() != N:
        raise ValueError(f"int8_matmul: scale has {scale.numel()} entries, expected N={N}")
    adt = dt_code(a.dtype, "int8_matmul")
    a, w_q = rows(a), rows(w_q)
    s, sdt = scale_vector(scale.reshape(-1).contiguous())
    c = torch.empty(M, N, dtype=a.dtype, device=dev)
    lib = kernels.lib()
    # fp32 activations with M >= 2 run on the matrix cores as bf16 hi + lo parts, split
    # into a workspace from torch's caching allocator; other calls need none
    need = lib.mls_wq_gemm_workspace(8, M, N, K, adt, 0)
    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    kernels.check(lib.mls_int8_gemm_ws(
        a.data_ptr(), adt, ld(a), w_q.data_ptr(), ld(w_q), s.data_ptr(), sdt,
        c.data_ptr(), adt, ld(c), M, N, K, ws.data_ptr() if need else None, need, stream(dev)), "int8_matmul")
    return c


def int8_dgrad(dy: torch.Tensor, w_q: torch.Tensor, scale: torch.Tensor):
    """dx [M, K] = (dy ∘ scale) [M, N] @ w_q [N, K]  (kernels/dequant_matmul.py:155-167)."""
    dev = require_hip("int8_dgrad", dy, w_q, scale)
    M, N = dy.shape
    K = w_q.shape[1]
    if w_q.dtype != torch.int8:
        raise TypeError(f"int8_dgrad: w_q must be int8, got {w_q.dtype}")
    if w_q.shape[0] != N:
        raise ValueError(f"int8_dgrad: w_q shape {tuple(w_q.shape)} does not match N={N}")
    if scale.numel() != N:
        raise ValueError(f"int8_dgrad: scale has {scale.numel()} entries, expected N={N}")
    ddt = dt_code(dy.dtype, "int8_dgrad")
    dy, w_q = rows(dy), rows(w_q)
    s, sdt = scale_vector(scale.reshape(-1).contiguous())
    dx = torch.empty(M, K, dtype=dy.dtype, device=dev)
    lib = kernels.lib()
    # 16-bit dy: the matrix-core route, with its scratch (scaled dy, transposed weights)
    # from torch's caching allocator; fp32 dy: the VALU kernel, no workspace
    need = lib.mls_int8_dgrad_workspace(M, N, K, ddt)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    kernels.check(lib.mls_int8_dgrad_ws(
        dy.data_ptr(), ddt, ld(dy), w_q.data_ptr(), ld(w_q), s.data_ptr(), sdt,
        dx.data_ptr(), ddt, ld(dx), M, N, K, ws.data_ptr(), need, stream(dev)), "int8_dgrad")
    return dx


def int4_matmul(a: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor,
                group_size: int):
    """a [M, K] @ dequant(int4-packed W [N, K/2], scales [N, K/group]).T
    (kernels/dequant_matmul.py:170-185)."""
    M, K = a.shape
    N = w_packed.shape[0]
    assert K % group_size == 0 and K == w_packed.shape[1] * 2
    dev = require_hip("int4_matmul", a, w_packed, scale)
    if w_packed.dtype != torch.uint8:
        raise TypeError(f"int4_matmul: w_packed must be uint8, got {w_packed.dtype}")
    G = K // group_size
    if scale.dim() != 2 or tuple(scale.shape) != (N, G):
        raise ValueError(f"int4_matmul: scale shape {tuple(scale.shape)}, expected {(N, G)}")
    adt = dt_code(a.dtype, "int4_matmul")
    a, w_packed = rows(a), rows(w_packed)
    if scale.dtype not in (torch.float32, torch.float16):
        scale = scale.to(torch.float32)
    sdt = dt_code(scale.dtype, "int4_matmul scale")
    c = torch.empty(M, N, dtype=a.dtype, device=dev)
    lib = kernels.lib()
    need = lib.mls_wq_gemm_workspace(4, M, N, K, adt, group_size)
    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    kernels.check(lib.mls_int4_gemm_ws(
        a.data_ptr(), adt, ld(a), w_packed.data_ptr(), ld(w_packed),
        scale.data_ptr(), sdt, scale.stride(0), scale.stride(1), group_size,
        c.data_ptr(), adt, ld(c), M, N, K, ws.data_ptr() if need else None, need, stream(dev)), "int4_matmul")
    return c
