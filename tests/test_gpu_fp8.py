"""gfx950 e4m3 GEMM vs the decode-then-fp32-matmul oracle.

The default datapath (bf16 MFMA on exactly widened operands) is held to the
BASELINE tolerances. The native fp8-MFMA datapath (native=True) truncates each product
of a group of 8 toward zero at 2^-13 of the group's largest before adding them: it is
held to the same tolerance on data without outliers, to |Δ| <= 2^-9 max(|ref|, rms(ref))
on outlier-heavy data, and its group rounding is pinned by a known-answer test."""

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


@pytest.mark.parametrize("native", [False, True])
@pytest.mark.parametrize("M,N,K", [(64, 96, 128), (256, 256, 256), (300, 200, 384), (1024, 512, 1024),
                                   (17, 33, 192)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_mfma_paths(dev, M, N, K, out_dtype, native):
    ab, bb, sa, sb = _operands(M, N, K, M + N + K, per_row=False)
    out = fp8_matmul(ab.to(dev), bb.to(dev), sa, sb, out_dtype=out_dtype, native=native)
    assert out.dtype == out_dtype
    _check(out, ref.fp8_matmul(ab.numpy(), bb.numpy(), sa, sb), f"fp8 {M}x{N}x{K} native={native}")


def test_exact_partial_tile_run(dev):
    """The exact e4m3 kernel on 256-row tiles with 11 row tiles: in the tile order, runs of
    4, 4 and 3 row tiles sweep the column tiles."""
    M, N, K = 2800, 8192, 256
    ab, bb, sa, sb = _operands(M, N, K, 11, per_row=False)
    out = fp8_matmul(ab.to(dev), bb.to(dev), sa, sb, out_dtype=torch.float32)
    _check(out, ref.fp8_matmul(ab.numpy(), bb.numpy(), sa, sb), f"fp8 {M}x{N}x{K} exact")


@pytest.mark.parametrize("M,N,K", [(64, 96, 128), (300, 200, 384), (5, 7, 48)])
def test_per_row_scales_with_outliers(dev, M, N, K):
    ab, bb, sa, sb = _operands(M, N, K, 3 * M + N, per_row=True, outliers=True)
    want = ref.fp8_matmul(ab.numpy(), bb.numpy(), sa.numpy(), sb.numpy())
    out = fp8_matmul(ab.to(dev), bb.to(dev), sa.to(dev), sb.to(dev), out_dtype=torch.float32)
    _check(out, want, "per-row exact")
    nat = fp8_matmul(ab.to(dev), bb.to(dev), sa.to(dev), sb.to(dev), out_dtype=torch.float32, native=True)
    ok, worst = ref.close_fp32(nat.cpu().numpy(), want)
    assert ok, f"per-row native: worst {worst:.3g}"


def test_exact_path_widens_every_byte(dev):
    """Every finite e4m3 byte goes through the hardware e4m3 -> bf16 widening of the
    exact datapath: A = the 254 finite bytes, B = identity, C = their values."""
    codes = np.array([b for b in range(256) if b & 0x7F != 0x7F], dtype=np.uint8)
    K = 256
    a = np.zeros((64, K), np.uint8)
    a[0, :len(codes)] = codes
    b = np.zeros((K, K), np.uint8)
    b[np.arange(K), np.arange(K)] = 0x38                        # e4m3 1.0
    out = fp8_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), 1.0, 1.0)
    got = out[0, :len(codes)].cpu().numpy()
    assert np.array_equal(got, ref.e4m3_decode(codes))   # -0.0 sums to +0.0


def test_native_group_rounding_known_answer(dev):
    """The fp8 MFMA aligns the 8 products of a group (k = 8i .. 8i + 7) to the largest and
    truncates each toward zero at 2^-13 of it (2^3 next to 256*256) before adding them:
    256*256 + 1*1 and 256*256 - 1*1 in one group lose the 1, +-9 keeps +-8, four 1s are
    lost one by one; in the next group the 1 survives. The default datapath keeps them."""
    K = 128

    def native(vals, native=True):
        a = np.zeros((64, K), np.float32)
        b = np.zeros((64, K), np.float32)
        for k, (x, y) in vals.items():
            a[:, k], b[:, k] = x, y
        A = torch.from_numpy(ref.e4m3_encode(a)).to(dev)
        B = torch.from_numpy(ref.e4m3_encode(b)).to(dev)
        return float(fp8_matmul(A, B, 1.0, 1.0, native=native, out_dtype=torch.float32)[0, 0])

    big = (256.0, 256.0)
    assert native({0: big, 1: (1.0, 1.0)}) == 65536.0
    assert native({0: big, 7: (1.0, 1.0)}) == 65536.0
    assert native({0: big, 8: (1.0, 1.0)}) == 65537.0
    assert native({0: big, 1: (-1.0, 1.0)}) == 65536.0       # toward zero, not -inf
    assert native({0: (-256.0, 256.0), 1: (1.0, 1.0)}) == -65536.0
    assert native({0: big, 1: (9.0, 1.0)}) == 65544.0
    assert native({0: big, 1: (-9.0, 1.0)}) == 65528.0
    assert native({0: big, 1: (1.0, 1.0), 2: (1.0, 1.0), 3: (1.0, 1.0), 4: (1.0, 1.0)}) == 65536.0
    assert native({0: big, 8: (-1.0, 1.0)}) == 65535.0
    assert native({0: big, 1: (-1.0, 1.0)}, native=False) == 65535.0


def _config_d(dev):
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
    da = ab.view(torch.float8_e4m3fn).float()
    db = bb.view(torch.float8_e4m3fn).float()
    want = (da @ db.t().contiguous()) * (sa[:, None] * sb[None, :])
    return ab, bb, sa, sb, want


def test_config_d(dev):
    """A [4096, 8192], B [8192, 8192], 1% outliers x20, per-row
    e4m3 scales, bf16 output; every output vs torch fp32 matmul of the decoded operands
    (rtol = atol = 1e-2), sampled rows vs the CPU oracle."""
    ab, bb, sa, sb, want = _config_d(dev)
    out = fp8_matmul(ab, bb, sa, sb, out_dtype=torch.bfloat16)
    rows = [0, 2049, 4095]
    _check(out[rows], ref.fp8_matmul(ab[rows].cpu().numpy(), bb.cpu().numpy(), sa[rows].cpu().numpy(),
                                     sb.cpu().numpy()), "config D rows")
    err = (out.float() - want).abs() - (1e-2 + 1e-2 * want.abs())
    worst = int(err.argmax())
    m, n = divmod(worst, want.shape[1])
    assert float(err.max()) <= 0, (f"config D worst excess {float(err.max()):.3g} at ({m}, {n}): "
                                   f"out {float(out[m, n]):.6g} want {float(want[m, n]):.6g}")


def test_config_d_native_error_bound(dev):
    """Config D on the fp8 matrix cores: within 2^-9 max(|ref|, rms(ref)) everywhere."""
    ab, bb, sa, sb, want = _config_d(dev)
    out = fp8_matmul(ab, bb, sa, sb, out_dtype=torch.float32, native=True)
    rms = float(want.pow(2).mean().sqrt())
    excess = (out - want).abs() - 2.0 ** -9 * torch.maximum(want.abs(), torch.tensor(rms, device=dev))
    assert float(excess.max()) <= 0, f"native config D excess {float(excess.max()):.3g} (rms {rms:.4g})"
