"""FP8 training's backward on the GPU (train/fp8.py:80-95): the e5m2 encoder
(bit-exact), the byte transpose (exact), the fp8 GEMM with an e5m2 A operand, and
FP8Linear's kernel backward against the reference's fp32 emulation.

Tolerances: fp32 outputs |Δ| <= 2^-9 max(|ref|, rms(ref)) (ref.close_fp32), 16-bit
outputs rtol = atol = 1e-2 (ref.close_bf16), against the decode-then-fp64 oracle. The
exact datapath widens e5m2 and e4m3 to bf16 without rounding, so it differs from the
oracle by summation order only."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import ref

from kernels.fp8_matmul import E4M3_MAX, E5M2_MAX, fp8_matmul, quantize_e5m2, transpose_u8
from train.fp8 import FP8Linear

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _boundaries():
    v = ref._POS5_VALUES.astype(np.float64)
    mids = (v[:-1] + v[1:]) / 2
    pts = np.concatenate([v, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                          np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
                          [60000.0, 61440.0, 1e9, 2.0 ** -17, 3 * 2.0 ** -17]]).astype(np.float32)
    return np.concatenate([pts, -pts, np.array([np.nan, -np.nan, np.inf, -np.inf], np.float32)])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [1.0, 0.37, 2.5e-6])
def test_quantize_e5m2_bit_exact(dev, dtype, scale):
    g = np.random.default_rng(int(scale * 1e6) + 3)
    x = np.concatenate([_boundaries() * np.float32(scale),
                        (g.standard_normal(100003) * 1e3 * scale).astype(np.float32)])
    xt = torch.from_numpy(x).to(dtype)
    got = quantize_e5m2(xt.to(dev), scale).cpu().numpy()
    want = ref.quantize_e5m2(xt.float().numpy(), scale)
    assert np.array_equal(got, want)


def test_quantize_e5m2_strided_rows(dev):
    g = torch.Generator().manual_seed(4)
    full = torch.randn(37, 130, generator=g) * 100
    x = full[:, 3:101]
    got = quantize_e5m2(full.to(dev)[:, 3:101], 0.01).cpu().numpy()
    assert np.array_equal(got, ref.quantize_e5m2(x.contiguous().numpy(), 0.01))


@pytest.mark.parametrize("R,C,off", [(1, 1, 0), (64, 64, 0), (63, 65, 0), (1000, 37, 0),
                                     (4096, 512, 0), (384, 256, 0), (300, 4096, 16), (130, 300, 5)])
def test_transpose_u8(dev, R, C, off):
    g = torch.Generator().manual_seed(R * C)
    full = torch.randint(0, 256, (R, C + off), generator=g, dtype=torch.uint8)
    t = full[:, off:] if off else full
    got = transpose_u8(full.to(dev)[:, off:] if off else full.to(dev))
    assert got.shape == (C, R) and got.is_contiguous()
    assert torch.equal(got.cpu(), t.t().contiguous())


def test_every_e5m2_byte_widens(dev):
    """Every finite e5m2 byte through the exact datapath's e5m2 -> bf16 widening:
    A = the 248 finite bytes, B = identity (e4m3 1.0), C = their values."""
    codes = np.array([b for b in range(256) if (b & 0x7F) < 0x7C], dtype=np.uint8)
    K = 256
    a = np.zeros((64, K), np.uint8)
    a[0, :len(codes)] = codes
    b = np.zeros((K, K), np.uint8)
    b[np.arange(K), np.arange(K)] = 0x38
    out = fp8_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), 1.0, 1.0, a_format="e5m2")
    assert np.array_equal(out[0, :len(codes)].cpu().numpy(), ref.e5m2_decode(codes))


def _operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g) * 1e-3          # gradient-like magnitudes
    b = torch.randn(N, K, generator=g)
    sa = float(a.abs().amax()) / E5M2_MAX
    sb = float(b.abs().amax()) / E4M3_MAX
    ab = ref.quantize_e5m2(a.numpy(), sa)
    bb = ref.quantize_e4m3(b.numpy(), sb)
    want = (ref.e5m2_decode(ab).astype(np.float64) * np.float32(sa)) @ \
        (ref.e4m3_decode(bb, nan_to_zero=False).astype(np.float64) * np.float32(sb)).T
    return torch.from_numpy(ab), torch.from_numpy(bb), sa, sb, want


@pytest.mark.parametrize("native", [False, True])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (300, 200, 384), (1024, 512, 2048), (17, 33, 40)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_e5m2_gemm_paths(dev, M, N, K, native, out_dtype):
    ab, bb, sa, sb, want = _operands(M, N, K, M + 7 * N + K)
    out = fp8_matmul(ab.to(dev), bb.to(dev), sa, sb, out_dtype, native=native, a_format="e5m2")
    o = out.float().cpu().numpy()
    ok, worst = ref.close_fp32(o, want) if out_dtype == torch.float32 else ref.close_bf16(o, want)
    assert ok, f"e5m2 x e4m3 {M}x{N}x{K} native={native}: worst {worst:.3g}"


def test_e5m2_gemm_rejects_bad_format(dev):
    ab, bb, sa, sb, _ = _operands(16, 16, 64, 1)
    with pytest.raises(ValueError, match="a_format"):
        fp8_matmul(ab.to(dev), bb.to(dev), sa, sb, a_format="e3m4")


@pytest.mark.parametrize("M,N,K", [(64, 128, 256), (300, 512, 192), (7, 24, 40)])
def test_fp8_linear_backward_kernel_vs_emulation(dev, M, N, K):
    """FP8Linear(use_kernel=True) backward (two e5m2 x e4m3 GEMMs + transposes) against
    the reference's emulation (use_kernel=False) on the same weights, inputs and
    upstream gradient; both against the oracle at the smallest shape."""
    torch.manual_seed(M + N + K)
    lin = nn.Linear(K, N, bias=False)
    mk, me = FP8Linear(lin, use_kernel=True).to(dev), FP8Linear(lin, use_kernel=False).to(dev)
    x = torch.randn(M, K, device=dev)
    dy = torch.randn(M, N, device=dev) * 1e-2
    grads = []
    for m in (mk, me):
        xi = x.clone().requires_grad_(True)
        m(xi).backward(dy)
        grads.append((xi.grad.float().cpu().numpy(), m.weight.grad.float().cpu().numpy()))
    (dxk, dwk), (dxe, dwe) = grads
    for got, want, what in ((dxk, dxe, "dx"), (dwk, dwe, "dw")):
        ok, worst = ref.close_fp32(got, want)
        assert ok, f"{what} {M}x{N}x{K}: worst {worst:.3g}"
    if M * N * K < 10000:
        # first call of the delayed scalers: just-in-time amax / fp8 max
        sx = max(float(x.abs().amax()), 1e-12) / E4M3_MAX
        sw = max(float(lin.weight.detach().abs().amax()), 1e-12) / E4M3_MAX
        sdy = max(float(dy.abs().amax()) / E5M2_MAX, 1e-12)
        xb = ref.quantize_e4m3(x.cpu().numpy(), sx)
        wb = ref.quantize_e4m3(lin.weight.detach().numpy(), sw)
        dx, dw = ref.fp8_linear_backward(dy.cpu().numpy(), xb, wb, sx, sw, sdy)
        for got, want, what in ((dxk, dx, "dx"), (dwk, dw, "dw")):
            ok, worst = ref.close_fp32(got, want)
            assert ok, f"{what} vs oracle: worst {worst:.3g}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_encoders_vector_path(dev, dtype, fmt):
    """Rows of a multiple of 4 elements take the 4-per-thread encoder: bit-exact too,
    including boundaries, NaN and per-row scales."""
    from kernels.fp8_matmul import quantize_e4m3
    g = np.random.default_rng(5)
    pts = _boundaries() if fmt == "e5m2" else np.concatenate(
        [ref._POS_VALUES, (ref._POS_VALUES[:-1] + ref._POS_VALUES[1:]) / 2]).astype(np.float32)
    x = np.concatenate([pts, -pts, (g.standard_normal(4096 * 4) * 50).astype(np.float32)])
    x = x[: (x.size // 256) * 256].reshape(-1, 256)
    xt = torch.from_numpy(x).to(dtype)
    enc = quantize_e5m2 if fmt == "e5m2" else quantize_e4m3
    want_fn = ref.quantize_e5m2 if fmt == "e5m2" else ref.quantize_e4m3
    assert np.array_equal(enc(xt.to(dev), 0.5).cpu().numpy(), want_fn(xt.float().numpy(), 0.5))
    rs = torch.rand(x.shape[0], 1, generator=torch.Generator().manual_seed(2)) + 0.1
    assert np.array_equal(enc(xt.to(dev), rs.to(dev)).cpu().numpy(), want_fn(xt.float().numpy(), rs.numpy()))


def test_fp8_linear_backward_config_d(dev):
    """FP8Linear's kernel backward at config D's shape (4096 tokens, 8192 -> 8192) against
    the reference's fp32 emulation of the same e4m3 / e5m2 operands (use_kernel=False,
    train/fp8.py:80-95) on the same weights, input and upstream gradient."""
    torch.manual_seed(9)
    M, N, K = 4096, 8192, 8192
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        lin = nn.Linear(K, N, bias=False)
        mk, me = FP8Linear(lin, use_kernel=True).to(dev), FP8Linear(lin, use_kernel=False).to(dev)
        g = torch.Generator(device=dev).manual_seed(10)
        x = torch.randn(M, K, generator=g, device=dev)
        dy = torch.randn(M, N, generator=g, device=dev) * 1e-2
        grads = []
        for m in (mk, me):
            xi = x.clone().requires_grad_(True)
            m(xi).backward(dy)
            grads.append((xi.grad.float(), m.weight.grad.float()))
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    (dxk, dwk), (dxe, dwe) = grads
    for got, want, what in ((dxk, dxe, "dx"), (dwk, dwe, "dw")):
        # |d| <= 2^-9 max(|want|, rms(want)), elementwise, as ref.close_fp32 states it
        bound = 2.0 ** -9 * torch.maximum(want.abs(), want.pow(2).mean().sqrt())
        excess = float(((got - want).abs() - bound).max())
        assert excess <= 0, f"{what} at config D's shape: worst excess {excess:.3g}"


@pytest.mark.parametrize("fmt", ["e5m2", "e4m3"])
@pytest.mark.parametrize("R,C,dtype,per_row,off", [
    (256, 512, torch.float32, False, 0),     # whole 64 x 64 tiles
    (130, 300, torch.float32, True, 0),      # ragged edge tiles, per-row scales
    (1, 1, torch.float32, False, 0),
    (64, 200, torch.bfloat16, False, 0),
    (200, 64, torch.float16, True, 0),
    (96, 128, torch.float32, False, 4),      # strided rows: the byte path for the input
    (4096, 8192, torch.float32, False, 0),   # config D's gradient
])
def test_quantize_fp8_t(dev, R, C, dtype, per_row, off, fmt):
    """One-pass encode + transpose: both outputs bit-identical to quantize_e5m2 /
    quantize_e4m3 and its byte transpose, boundaries, NaN and saturation included."""
    from kernels.fp8_matmul import quantize_e4m3, quantize_e4m3_t, quantize_e5m2_t
    enc_t, enc = (quantize_e5m2_t, quantize_e5m2) if fmt == "e5m2" else (quantize_e4m3_t, quantize_e4m3)
    oracle = ref.quantize_e5m2 if fmt == "e5m2" else ref.quantize_e4m3
    g = torch.Generator().manual_seed(R * 7 + C)
    x = torch.randn(R, C + off, generator=g) * 3e3
    pts = torch.from_numpy(_boundaries())
    n = min(pts.numel(), x.numel())
    x.view(-1)[:n] = pts[:n] * 1.7
    xd = x.to(dtype).to(dev)
    xs = xd[:, off:] if off else xd
    scale = (torch.rand(R, 1, generator=g) + 0.25).to(dev) if per_row else 0.37
    bits, bits_t = enc_t(xs, scale)
    want = enc(xs.contiguous(), scale)
    assert bits.shape == (R, C) and bits_t.shape == (C, R) and bits_t.is_contiguous()
    assert torch.equal(bits, want)
    assert torch.equal(bits_t, want.t().contiguous())
    if R * C <= 64 * 1024:
        sc = scale.cpu().numpy() if per_row else scale
        assert np.array_equal(bits.cpu().numpy(), oracle(xs.float().cpu().numpy(), sc))


def test_fp8_linear_no_grad_forward(dev):
    """Without gradients the kernel forward encodes once (no transposed copies) and gives
    the same output as the training forward, which writes both layouts."""
    torch.manual_seed(3)
    lin = nn.Linear(192, 320, bias=False)
    m = FP8Linear(lin, use_kernel=True).to(dev)
    x = torch.randn(2, 33, 192, device=dev)
    y_train = m(x.clone().requires_grad_(True)).detach()
    m2 = FP8Linear(lin, use_kernel=True).to(dev)
    with torch.no_grad():
        y_inf = m2(x)
    assert torch.equal(y_train, y_inf)


def _teacher_task(dev, d=64, classes=10, n=4096, seed=0):
    """Labels from a fixed random teacher: argmax of a random linear map of x."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(n, d, generator=g, device=dev)
    t = torch.randn(d, classes, generator=g, device=dev)
    return x, (x @ t).argmax(1)


def _train(model, x, y, steps=80, batch=64, lr=1e-3, seed=1):
    opt = torch.optim.Adam(model.parameters(), lr=lr)
    g = torch.Generator(device=x.device).manual_seed(seed)
    loss = None
    for _ in range(steps):
        idx = torch.randint(0, x.shape[0], (batch,), generator=g, device=x.device)
        loss = F.cross_entropy(model(x[idx]), y[idx])
        opt.zero_grad()
        loss.backward()
        opt.step()
    with torch.no_grad():
        return float(F.cross_entropy(model(x), y))


def test_fp8_training_converges_close_to_fp32(dev):
    """test_fp8.py:101-130 of the reference on this build's kernel path: the same network
    trained with FP8Linear(use_kernel=True) (e4m3 forward GEMM, e5m2 x e4m3 backward
    GEMMs, delayed scaling) ends within 15% of the fp32 run's loss."""
    x, y = _teacher_task(dev)
    torch.manual_seed(42)
    base = nn.Sequential(nn.Linear(64, 128, bias=False), nn.GELU(), nn.Linear(128, 128, bias=False),
                         nn.GELU(), nn.Linear(128, 10, bias=False)).to(dev)
    import copy
    fp32 = copy.deepcopy(base)
    fp8 = copy.deepcopy(base)
    for i in (0, 2, 4):
        fp8[i] = FP8Linear(fp8[i], enabled=True, use_kernel=True).to(dev)
    l32 = _train(fp32, x, y)
    l8 = _train(fp8, x, y)
    assert l8 < l32 * 1.15, f"fp8 {l8:.3f} vs fp32 {l32:.3f}"
