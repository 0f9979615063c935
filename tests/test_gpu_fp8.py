"""gfx950 e4m3 GEMM (native fp8 MFMA) vs the decode-then-fp32-matmul oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import ref

from kernels.fp8_matmul import E4M3_MAX, fp8_matmul, quantize_e4m3

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _check(out, want, what):
    o = out.float().cpu().numpy()
    ok, worst = ref.close_fp32(o, want) if out.dtype == torch.float32 else ref.close_bf16(o, want)
    assert ok, f"{what}: worst {worst:.3g}"


def test_reference_shapes_golden(dev):
    """test_fp8.py:39-48 shapes, per-tensor float scales, fp32 output."""
    d = golden("fp8_small")
    for t in ("t1", "t2", "t3"):
        out = fp8_matmul(torch.from_numpy(d[f"{t}_a"]).to(dev), torch.from_numpy(d[f"{t}_b"]).to(dev),
                         float(d[f"{t}_sa"]), float(d[f"{t}_sb"]))
        assert out.dtype == torch.float32
        _check(out, d[f"{t}_y"], t)


def _operands(M, N, K, seed, per_row, outliers=False):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g)
    b = torch.randn(N, K, generator=g)
    if outliers:
        a = torch.where(torch.rand(M, K, generator=g) < 0.01, a * 20, a)
        b = torch.where(torch.rand(N, K, generator=g) < 0.01, b * 20, b)
    if per_row:
        sa = a.abs().amax(dim=1) / E4M3_MAX
        sb = b.abs().amax(dim=1) / E4M3_MAX
        ab = torch.from_numpy(ref.quantize_e4m3(a.numpy(), sa[:, None].numpy()))
        bb = torch.from_numpy(ref.quantize_e4m3(b.numpy(), sb[:, None].numpy()))
    else:
        sa = float(a.abs().amax()) / E4M3_MAX
        sb = float(b.abs().amax()) / E4M3_MAX
        ab = torch.from_numpy(ref.quantize_e4m3(a.numpy(), sa))
        bb = torch.from_numpy(ref.quantize_e4m3(b.numpy(), sb))
    return ab, bb, sa, sb


@pytest.mark.parametrize("M,N,K", [(64, 96, 128), (256, 256, 256), (300, 200, 384), (1024, 512, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_mfma_path(dev, M, N, K, out_dtype):
    ab, bb, sa, sb = _operands(M, N, K, M + N + K, per_row=False)
    out = fp8_matmul(ab.to(dev), bb.to(dev), sa, sb, out_dtype=out_dtype)
    assert out.dtype == out_dtype
    _check(out, ref.fp8_matmul(ab.numpy(), bb.numpy(), sa, sb), f"fp8 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(64, 96, 128), (300, 200, 384), (5, 7, 48)])
def test_per_row_scales(dev, M, N, K):
    ab, bb, sa, sb = _operands(M, N, K, 3 * M + N, per_row=True, outliers=True)
    out = fp8_matmul(ab.to(dev), bb.to(dev), sa.to(dev), sb.to(dev), out_dtype=torch.float32)
    _check(out, ref.fp8_matmul(ab.numpy(), bb.numpy(), sa.numpy(), sb.numpy()), "per-row")


def test_zero_dim_tensor_scales(dev):
    ab, bb, sa, sb = _operands(128, 128, 256, 1, per_row=False)
    out = fp8_matmul(ab.to(dev), bb.to(dev), torch.tensor(sa, device=dev), torch.tensor(sb, device=dev))
    _check(out, ref.fp8_matmul(ab.numpy(), bb.numpy(), sa, sb), "0-d scales")


def test_quantize_then_matmul_on_device(dev):
    """quantize_e4m3 on the device feeds fp8_matmul (the FP8Linear forward)."""
    g = torch.Generator().manual_seed(4)
    a, b = torch.randn(128, 256, generator=g), torch.randn(192, 256, generator=g)
    sa, sb = float(a.abs().amax()) / E4M3_MAX, float(b.abs().amax()) / E4M3_MAX
    ab, bb = quantize_e4m3(a.to(dev), sa), quantize_e4m3(b.to(dev), sb)
    assert np.array_equal(ab.cpu().numpy(), ref.quantize_e4m3(a.numpy(), sa))
    _check(fp8_matmul(ab, bb, sa, sb), ref.fp8_matmul(ab.cpu().numpy(), bb.cpu().numpy(), sa, sb), "q+mm")


def test_config_d(dev):
    """A [4096, 8192], B [8192, 8192], 1% outliers x20, per-row
    e4m3 scales, bf16 output; every output vs torch fp32 matmul of the decoded operands,
    sampled rows vs the CPU oracle."""
    M, N, K = 4096, 8192, 8192
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(M, K, generator=g, device=dev)
    a = torch.where(torch.rand(M, K, generator=g, device=dev) < 0.01, a * 20, a)
    sa = a.abs().amax(dim=1) / E4M3_MAX
    ab = quantize_e4m3(a, sa[:, None])
    del a
    b = torch.randn(N, K, generator=g, device=dev)
    b = torch.where(torch.rand(N, K, generator=g, device=dev) < 0.01, b * 20, b)
    sb = b.abs().amax(dim=1) / E4M3_MAX
    bb = quantize_e4m3(b, sb[:, None])
    del b
    out = fp8_matmul(ab, bb, sa, sb, out_dtype=torch.bfloat16)
    da = ab.view(torch.float8_e4m3fn).float()
    db = bb.view(torch.float8_e4m3fn).float()
    want = (da @ db.t().contiguous()) * (sa[:, None] * sb[None, :])
    err = (out.float() - want).abs() - (1e-2 + 1e-2 * want.abs())
    assert float(err.max()) <= 0, f"config D worst excess {float(err.max()):.3g}"
    rows = [0, 2049, 4095]
    _check(out[rows], ref.fp8_matmul(ab[rows].cpu().numpy(), bb.cpu().numpy(), sa[rows].cpu().numpy(),
                                     sb.cpu().numpy()), "config D rows")
