"""Shapes at the 32-bit offset limits of the fast kernels.

Each fast path addresses its operands through 32-bit buffer offsets and refuses a shape
whose offsets would not fit, handing the call to a kernel with 64-bit indexing. These
tests put each limit between two calls, one just below it (the fast kernel runs) and
one just above (the fallback runs), and check both against torch fp32 of the decoded
operands on the device:

  - medium GEMM (csrc/gemm_small.hip): M * lda * 2 bytes of x below 2^29;
  - skinny GEMM (csrc/gemv_mfma.hip): 16 rows of x, 16 * lda * 2 bytes, below 2^31;
  - MFMA engine (csrc/gemm_mfma16.hip): 256 * lda * 2 bytes (the tallest tile) below 2^31,
    checked whatever tile height the shape then gets (16 rows here);
  - e4m3 GEMM (csrc/gemm_fp8.hip): 256 * lda bytes below 2^31, likewise.

The operands are generated on the device (several GB at these sizes), and the outputs,
a few thousand values, are compared on the host. Above each limit the fallback is the
one-thread-per-output kernel, which takes seconds at these K (16 s for the skinny case).
A kernel trace of this file shows gemm_small / gemv_mfma / mfma16_gemm below the limits
and the generic kernels above them.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref

from kernels.dequant_matmul import int4_matmul, int8_matmul
from kernels.fp8_matmul import decode_e4m3, fp8_matmul, quantize_e4m3
from serve.quantize import dequantize_int4, quantize_int4, quantize_int8

pytestmark = pytest.mark.gpu


def _check(out: torch.Tensor, want: torch.Tensor, what: str):
    ok, worst = ref.close_bf16(out.float().cpu().numpy(), want.float().cpu().numpy())
    assert ok, f"{what}: worst {worst:.3g}"


def _act(M, K, dev, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(M, K, generator=g, device=dev).to(dtype)


def _int8(N, K, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)


def _ref_int8(a, q, s):
    return a.float() @ (q.float() * s.float()[:, None]).t()


@pytest.mark.parametrize("K", [6_710_784, 6_710_912])  # M * K * 2 just below / at 2^29 + 256
def test_medium_gemm_x_limit(dev, K):
    M, N = 40, 8
    assert (M * K * 2 < 2 ** 29) == (K == 6_710_784)
    a = _act(M, K, dev, 1)
    q, s = _int8(N, K, dev, 2)
    _check(int8_matmul(a, q, s), _ref_int8(a, q, s), f"medium int8 K={K}")


@pytest.mark.parametrize("K", [2 ** 26 - 128, 2 ** 26])  # 16 rows of x: 16 * K * 2 below / at 2^31
def test_skinny_gemm_x_limit(dev, K):
    M, N, gs = 2, 16, 128
    a = _act(M, K, dev, 3)
    g = torch.Generator(device=dev).manual_seed(4)
    p, s = quantize_int4(torch.randn(N, K, generator=g, device=dev) * 0.02, gs)
    s16 = s.to(torch.float16)
    want = a.float() @ dequantize_int4(p, s16.float(), gs).t()
    _check(int4_matmul(a, p, s16, gs), want, f"skinny int4 K={K}")


@pytest.mark.parametrize("K", [4_194_240, 4_194_304])  # 256 rows of x: 256 * K * 2 below / at 2^31
def test_engine_tile_limit(dev, K):
    M, N = 300, 256
    a = _act(M, K, dev, 5)
    q, s = _int8(N, K, dev, 6)
    _check(int8_matmul(a, q, s), _ref_int8(a, q, s), f"engine int8 K={K}")


@pytest.mark.parametrize("K", [8_388_544, 8_388_608])  # 256 rows of e4m3: 256 * K below / at 2^31
def test_fp8_tile_limit(dev, K):
    M, N = 64, 64
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn(M, K, generator=g, device=dev)
    b = torch.randn(N, K, generator=g, device=dev)
    sa, sb = float(a.abs().amax()) / 448.0, float(b.abs().amax()) / 448.0
    ab, bb = quantize_e4m3(a, sa), quantize_e4m3(b, sb)
    del a, b
    want = (decode_e4m3(ab) @ decode_e4m3(bb).t()) * (sa * sb)
    _check(fp8_matmul(ab, bb, sa, sb, out_dtype=torch.bfloat16), want, f"fp8 K={K}")
