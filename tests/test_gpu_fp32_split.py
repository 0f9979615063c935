"""fp32 activations on the matrix cores (the reference's engine runs fp32 end to end,
serve/engine.py:166, so every QuantLinear call there carries fp32 x): with M >= 2, x is
split into bf16 hi + lo parts and both are multiplied on the bf16 MFMA with fp32
accumulation and added in fp32.

Bound: BASELINE's fp32 rule, |d| <= 2^-9 max(|ref|, rms(ref)) against the dequantize-
then-fp32-matmul oracle (the split itself keeps x to ~2^-16). Full-size shapes compare
every output with torch's fp32 matmul of the dequantized weights on the GPU (TF32 off) and
sampled rows with the CPU oracle; small shapes compare everything with the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref

from kernels.dequant_matmul import int4_matmul, int8_dgrad, int8_matmul
from serve.quantize import quantize_int4, quantize_int8

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _check32(out, want, what):
    assert out.dtype == torch.float32
    ok, worst = ref.close_fp32(out.cpu().numpy(), want)
    assert ok, f"{what}: worst {worst:.3g} of the fp32 bound"


def _rule32(out, want, what):
    """The fp32 rule on every output against a GPU fp32 reference."""
    o, w = out.float(), want.float()
    rms = float(w.double().pow(2).mean().sqrt())
    ratio = (o - w).abs() / ((2.0 ** -9) * torch.clamp(w.abs(), min=rms))
    worst = float(ratio.max())
    assert worst <= 1.0, f"{what}: worst {worst:.3g} of the fp32 bound"
    return worst


def _deq8(q, s):
    return q.float() * s.float()[:, None]


def _deq4(p, s, gs):
    N = p.shape[0]
    w = torch.stack(((p & 15).float() - 8.0, (p >> 4).float() - 8.0), dim=-1).reshape(N, -1)
    return (w.reshape(N, -1, gs) * s.float()[:, :, None]).reshape(N, -1)


def test_config_c_fp32(dev):
    """Config C's shape (INT8, 2048 x 11008 x 4096, fp16 scales) with fp32 x, as the
    reference's engine would call it: every output within the fp32 rule."""
    M, N, K = 2048, 11008, 4096
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(M, K, generator=g, device=dev)
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
    s16 = s.to(torch.float16)
    out = int8_matmul(a, q, s16)
    assert out.dtype == torch.float32 and out.shape == (M, N)
    _rule32(out, a @ _deq8(q, s16).t(), "config C fp32")
    rows = [0, 1, 1023, 2047]
    _check32(out[rows], ref.int8_matmul(a[rows].cpu().numpy(), q.cpu().numpy(), s16.float().cpu().numpy()),
             "config C fp32 rows")


def test_int4_prefill_fp32(dev):
    """INT4 g128, 2048 x 4096 x 4096, fp32 x: every output within the fp32 rule."""
    M, N, K, gs = 2048, 4096, 4096, 128
    g = torch.Generator(device=dev).manual_seed(1)
    a = torch.randn(M, K, generator=g, device=dev)
    p, s = quantize_int4(torch.randn(N, K, generator=g, device=dev) * 0.02, gs)
    s16 = s.to(torch.float16)
    out = int4_matmul(a, p, s16, gs)
    _rule32(out, a @ _deq4(p, s16, gs).t(), "INT4 prefill fp32")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("M,N,K,gs", [
    (17, 256, 256, 128),    # one row past the GEMV range: medium GEMM on 64 split rows
    (31, 1000, 1088, 64),   # ragged N, 17 steps, groups of 64
    (64, 4096, 4096, 128),  # an engine prefill chunk: medium GEMM
    (100, 333, 640, 128),   # odd N
    (200, 520, 768, 256),   # 448 split rows: medium GEMM, a group spans two steps
    (300, 1000, 512, 64),   # 640 split rows: the engine on 128-row tiles (INT8: 256)
    (513, 768, 640, 128),   # one row past a 512-row boundary
])
def test_fp32_split_shapes(dev, bits, M, N, K, gs):
    g = torch.Generator().manual_seed(M * 7 + N + bits)
    a = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    if bits == 8:
        q, s = quantize_int8(w)
        out = int8_matmul(a.to(dev), q.to(dev), s.to(dev))
        want = ref.int8_matmul(a.numpy(), q.numpy(), s.numpy())
    else:
        q, s = quantize_int4(w, gs)
        out = int4_matmul(a.to(dev), q.to(dev), s.to(dev), gs)
        want = ref.int4_matmul(a.numpy(), q.numpy(), s.numpy(), gs)
    assert out.shape == (M, N)
    _check32(out, want, f"fp32 split int{bits} M={M} N={N} K={K}")


def test_fp32_split_strided_unaligned_and_f16_scales(dev):
    """x rows 4 floats past a 16-byte boundary (the split pass's element-wise loads), a row
    stride above K, fp16 scales; INT8 and INT4."""
    M, N, K, gs = 40, 640, 1024, 128
    g = torch.Generator().manual_seed(5)
    wide = torch.randn(M, K + 9, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    xv = wide.to(dev)[:, 1:K + 1]  # lda = K + 9, 4-byte offset
    xs = wide[:, 1:K + 1].numpy()
    q, s = quantize_int8(w.to(dev))
    s16 = s.to(torch.float16)
    _check32(int8_matmul(xv, q, s16), ref.int8_matmul(xs, q.cpu().numpy(), s16.float().cpu().numpy()), "int8")
    p4, s4 = quantize_int4(w.to(dev), gs)
    s4 = s4.to(torch.float16)
    _check32(int4_matmul(xv, p4, s4, gs), ref.int4_matmul(xs, p4.cpu().numpy(), s4.float().cpu().numpy(), gs),
             "int4")


def test_fp32_split_keeps_precision_beyond_bf16(dev):
    """Inputs whose low mantissa bits matter: x = 1 + 2^-12 k patterns that bf16 alone
    would round away. The split result stays within 2^-14 of the fp32 oracle, far below
    what a single bf16 rounding of x (2^-9) gives."""
    M, N, K = 64, 256, 512
    g = torch.Generator().manual_seed(9)
    a = 1.0 + torch.randint(0, 4096, (M, K), generator=g).float() * 2.0 ** -12
    a = a * torch.where(torch.rand(M, K, generator=g) < 0.5, -1.0, 1.0)
    q, s = quantize_int8(torch.randn(N, K, generator=g) * 0.02)
    out = int8_matmul(a.to(dev), q.to(dev), s.to(dev)).cpu().numpy()
    want = ref.int8_matmul(a.numpy(), q.numpy(), s.numpy()).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    assert np.abs(out - want).max() <= 2.0 ** -14 * max(rms, np.abs(want).max())


def test_fp32_split_nonfinite(dev):
    """An inf or NaN in x reaches the outputs as in fp32 arithmetic: the same outputs are
    infinite / NaN as torch's fp32 matmul of the dequantized weights gives."""
    M, N, K = 32, 256, 256
    g = torch.Generator(device=dev).manual_seed(3)
    a = torch.randn(M, K, generator=g, device=dev)
    a[3, 17] = float("inf")
    a[7, 5] = float("-inf")
    a[20, 100] = float("nan")
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
    out = int8_matmul(a, q, s)
    want = a @ _deq8(q, s).t()
    assert torch.equal(torch.isnan(out), torch.isnan(want))
    assert torch.equal(torch.isposinf(out), torch.isposinf(want))
    assert torch.equal(torch.isneginf(out), torch.isneginf(want))
    fin = torch.isfinite(want)
    _rule32(out[fin], want[fin], "finite outputs next to non-finite ones")


def test_fp32_small_m_unchanged(dev):
    """M = 1 asks for no workspace (INT8: the VALU GEMV with fp32 FMAs; INT4: the LDS GEMV
    splitting x in registers); from M = 2 on the split rows are 32 per 16 rows of x (used by
    the split pass where the skinny kernel cannot split x itself)."""
    import kernels
    L = kernels.lib()
    assert L.mls_wq_gemm_workspace(8, 1, 4096, 4096, kernels.MLS_F32, 0) == 0
    assert L.mls_wq_gemm_workspace(8, 16, 4096, 4096, kernels.MLS_F32, 0) == 32 * 4096 * 2
    assert L.mls_wq_gemm_workspace(8, 17, 4096, 4096, kernels.MLS_F32, 0) == 64 * 4096 * 2
    assert L.mls_wq_gemm_workspace(8, 2048, 4096, 4096, kernels.MLS_BF16, 0) == 0
    assert L.mls_wq_gemm_workspace(4, 64, 4096, 4096, kernels.MLS_F32, 32) == 0  # groups of 32: VALU
    M, N, K = 1, 1000, 1024
    g = torch.Generator().manual_seed(4)
    a = torch.randn(M, K, generator=g)
    q, s = quantize_int8(torch.randn(N, K, generator=g) * 0.02)
    _check32(int8_matmul(a.to(dev), q.to(dev), s.to(dev)), ref.int8_matmul(a.numpy(), q.numpy(), s.numpy()), "M=1")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("M,N,K,gs", [
    (2, 4096, 4096, 128),   # speculative verify with one draft token
    (5, 4096, 4096, 128),   # verify with gamma = 4, or a decode batch of 5
    (16, 1000, 1152, 128),  # ragged N, 9 steps
    (7, 333, 768, 256),     # odd M, ragged N, a group of two steps
    (3, 520, 1088, 64),     # groups of 64: 64-k steps
    (16, 512, 14336, 128),  # long K: 16 wavefronts
])
def test_fp32_split_skinny(dev, bits, M, N, K, gs):
    """2 <= M <= 16 with fp32 x: the skinny MFMA GEMV runs every x MFMA on the hi and the lo
    part into one accumulator."""
    g = torch.Generator().manual_seed(M * 13 + N + bits)
    a = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    if bits == 8:
        q, s = quantize_int8(w)
        out = int8_matmul(a.to(dev), q.to(dev), s.to(torch.float16).to(dev))
        want = ref.int8_matmul(a.numpy(), q.numpy(), s.to(torch.float16).float().numpy())
    else:
        q, s = quantize_int4(w, gs)
        out = int4_matmul(a.to(dev), q.to(dev), s.to(dev), gs)
        want = ref.int4_matmul(a.numpy(), q.numpy(), s.numpy(), gs)
    _check32(out, want, f"fp32 skinny int{bits} M={M} N={N} K={K}")


@pytest.mark.parametrize("bits", [8, 4])
def test_fp32_skinny_without_workspace(dev, bits):
    """2 <= M <= 16 with fp32 x splits x inside the skinny kernel, so the entry points without a
    workspace (mls_int8_gemm / mls_int4_gemm) take the matrix cores too, with the same outputs
    as the workspace entry points; x whose rows the kernel cannot load as 16-byte pieces (an odd
    row stride) takes the split pass, under the same rule."""
    import kernels
    from kernels._hip import stream
    M, N, K, gs = 5, 1000, 2048, 128
    g = torch.Generator().manual_seed(55 + bits)
    a = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    L = kernels.lib()
    ad = a.to(dev)
    c = torch.empty(M, N, dtype=torch.float32, device=dev)
    if bits == 8:
        q, s = quantize_int8(w.to(dev))
        s = s.to(torch.float16)
        rc = L.mls_int8_gemm(ad.data_ptr(), kernels.MLS_F32, K, q.data_ptr(), K, s.data_ptr(), kernels.MLS_F16,
                             c.data_ptr(), kernels.MLS_F32, N, M, N, K, stream(dev))
        via_ws = int8_matmul(ad, q, s)
        want = ref.int8_matmul(a.numpy(), q.cpu().numpy(), s.float().cpu().numpy())
    else:
        q, s = quantize_int4(w.to(dev), gs)
        rc = L.mls_int4_gemm(ad.data_ptr(), kernels.MLS_F32, K, q.data_ptr(), K // 2, s.data_ptr(), kernels.MLS_F32,
                             s.stride(0), 1, gs, c.data_ptr(), kernels.MLS_F32, N, M, N, K, stream(dev))
        via_ws = int4_matmul(ad, q, s, gs)
        want = ref.int4_matmul(a.numpy(), q.cpu().numpy(), s.cpu().numpy(), gs)
    torch.cuda.synchronize(dev)
    assert rc == 0
    assert torch.equal(c, via_ws)
    _check32(c, want, f"fp32 M={M} int{bits}, no workspace")
    # row stride K + 1 floats: not a whole number of 16-byte pieces per row
    big = torch.zeros(M, K + 1, dtype=torch.float32, device=dev)
    big[:, :K] = ad
    xs = big[:, :K]
    out = int8_matmul(xs, q, s) if bits == 8 else int4_matmul(xs, q, s, gs)
    _check32(out, want, f"fp32 M={M} int{bits}, odd row stride")


@pytest.mark.parametrize("M,K,pad", [
    (1, 8192, 0),   # 1 weight row per wavefront, 8 chunks per lane: one partial per lane
    (1, 4096, 0),   # 2 rows: 2 partials
    (1, 2048, 0),   # 4 rows: 4 partials
    (1, 1024, 0),   # 8 rows: 8 partials
    (2, 1008, 1),   # K % 64 != 0 (no matrix-core path), x rows K + 1 apart: 2 x 8 = 16 partials
    (3, 1008, 0),   # 4 rows of x per block (the last repeats row 2) x 8 = 32 partials
])
def test_fp32_register_gemv_reduction_depths(dev, M, K, pad):
    """INT8 with fp32 x on the register GEMV (M = 1, or K that the matrix-core paths do not
    take): every number of per-lane partials its butterfly reduces, the lane-half and
    16-lane-row steps as swaps, against the oracle under the fp32 rule (ragged N)."""
    N = 1000
    g = torch.Generator(device="cpu").manual_seed(4000 + K + M)
    a = torch.randn(M, K + pad, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    q, s = quantize_int8(w.to(dev))
    ax = a.to(dev)[:, :K]
    out = int8_matmul(ax, q, s)
    assert out.shape == (M, N)
    _check32(out, ref.int8_matmul(a[:, :K].numpy(), q.cpu().numpy(), s.float().cpu().numpy()),
             f"register GEMV fp32 INT8 M={M} K={K}")


def test_int8_dgrad_fp32_training_shape(dev):
    """The INT8 STE input gradient with fp32 dy at a training shape (4096 x 11008 -> 4096):
    ys = dy * s in fp32 split into hi + lo rows on the matrix cores. Every output within
    the fp32 rule against torch fp32 of (dy * s) @ W_q on the GPU."""
    M, N, K = 4096, 11008, 4096
    g = torch.Generator(device=dev).manual_seed(8)
    dy = torch.randn(M, N, generator=g, device=dev)
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
    out = int8_dgrad(dy, q, s)
    assert out.dtype == torch.float32 and out.shape == (M, K)
    _rule32(out, (dy * s[None, :]) @ q.float(), "dgrad fp32 training shape")
    rows = [0, 2049, 4095]
    _check32(out[rows], ref.int8_dgrad(dy[rows].cpu().numpy(), q.cpu().numpy(), s.cpu().numpy()), "dgrad rows")


def test_ws_entry_points_reject_short_workspace(dev):
    """The workspace entry points check the workspace they are given before any launch."""
    import kernels
    L = kernels.lib()
    M, N, K = 64, 256, 512
    a = torch.randn(M, K, device=dev)
    q = torch.zeros(N, K, dtype=torch.int8, device=dev)
    s = torch.ones(N, device=dev)
    c = torch.empty(M, N, device=dev)
    need = L.mls_wq_gemm_workspace(8, M, N, K, kernels.MLS_F32, 0)
    assert need == 64 * 2 * K * 2
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = L.mls_int8_gemm_ws(a.data_ptr(), kernels.MLS_F32, K, q.data_ptr(), K, s.data_ptr(), kernels.MLS_F32,
                            c.data_ptr(), kernels.MLS_F32, N, M, N, K, ws.data_ptr(), need - 1, st)
    assert rc == kernels.MLS_ERR_ARG
    rc = L.mls_int8_gemm_ws(a.data_ptr(), kernels.MLS_F32, K, q.data_ptr(), K, s.data_ptr(), kernels.MLS_F32,
                            c.data_ptr(), kernels.MLS_F32, N, M, N, K, None, 0, st)
    assert rc == kernels.MLS_ERR_ARG
