"""gfx950 INT8 / INT4 weight-only GEMMs vs the dequantize-then-fp32-matmul oracle.

Tolerances (BASELINE): fp32 outputs |Δ| <= 2^-9 max(|ref|, rms(ref)); bf16 and fp16
outputs rtol = atol = 1e-2. Full-size configs compare every output against torch's
fp32 matmul of the dequantized weights on the GPU (a floating-point reference of
the same op, TF32 off) and sampled rows against the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import ref

from kernels.dequant_matmul import int4_matmul, int8_dgrad, int8_matmul
from serve.quantize import quantize_int4, quantize_int8

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _check(out: torch.Tensor, want: np.ndarray, what: str):
    o = out.float().cpu().numpy()
    if out.dtype == torch.float32:
        ok, worst = ref.close_fp32(o, want)
    else:
        ok, worst = ref.close_bf16(o, want)
    assert ok, f"{what}: worst {worst:.3g} (max |Δ| {np.abs(o - want).max():.3g})"


def _data(M, N, K, seed, wscale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g), torch.randn(N, K, generator=g) * wscale


# --------------------------------------------------------------- reference test shapes (fp32)

@pytest.mark.parametrize("M,N,K", [(4, 32, 48), (17, 33, 64), (1, 64, 32), (33, 256, 512)])
def test_int8_reference_shapes(dev, M, N, K):
    a, w = _data(M, N, K, M * 1000 + N)
    q, s = quantize_int8(w)
    out = int8_matmul(a.to(dev), q.to(dev), s.to(dev))
    assert out.dtype == torch.float32 and out.shape == (M, N)
    _check(out, ref.int8_matmul(a.numpy(), q.numpy(), s.numpy()), "int8")


@pytest.mark.parametrize("M,N,K,gs", [(4, 32, 64, 16), (9, 33, 32, 16), (1, 16, 64, 32),
                                      (33, 256, 512, 64), (3, 40, 512, 128)])
def test_int4_reference_shapes(dev, M, N, K, gs):
    a, w = _data(M, N, K, M * 1000 + N + gs)
    p, s = quantize_int4(w, gs)
    out = int4_matmul(a.to(dev), p.to(dev), s.to(dev), gs)
    _check(out, ref.int4_matmul(a.numpy(), p.numpy(), s.numpy(), gs), "int4")


def test_int4_golden_fixture(dev):
    d = golden("gemm_int4_small")
    for t in ("t1", "t2", "t3", "g128"):
        gs = int(d[f"{t}_gs"])
        out = int4_matmul(torch.from_numpy(d[f"{t}_a"]).to(dev), torch.from_numpy(d[f"{t}_packed"]).to(dev),
                          torch.from_numpy(d[f"{t}_scale"]).to(dev), gs)
        _check(out, d[f"{t}_y"], t)


def test_config_a_golden(dev):
    """INT8, x fp32 [8, 512], W [2048, 512], seed 0."""
    d = golden("gemm_int8_config_a")
    out = int8_matmul(torch.from_numpy(d["x"]).to(dev), torch.from_numpy(d["w_q"]).to(dev),
                      torch.from_numpy(d["scale"]).to(dev))
    _check(out, d["y"], "config A")


# --------------------------------------------------------------- decode configs (bf16)

def _int4_setup(dev, M, N, K, gs, seed, dtype=torch.bfloat16):
    a, w = _data(M, N, K, seed, 0.02)
    p, s = quantize_int4(w.to(dev), gs)
    s16 = s.to(torch.float16)
    ab = a.to(dtype)
    want = ref.int4_matmul(ab.float().numpy(), p.cpu().numpy(), s16.float().cpu().numpy(), gs)
    return ab.to(dev), p, s16, want


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16])
def test_config_b_int4_gemv(dev, M):
    """INT4 g128, K = N = 4096, bf16 x, fp16 scales, M in {1, 4, 16}."""
    a, p, s, want = _int4_setup(dev, M, 4096, 4096, 128, 100 + M)
    out = int4_matmul(a, p, s, 128)
    assert out.dtype == torch.bfloat16
    _check(out, want, f"config B M={M}")


@pytest.mark.parametrize("bits,N,K,dtype,sdt,pad", [
    (4, 1000, 4096, torch.bfloat16, torch.float16, 64),   # ragged N, x rows 64 elements apart
    (4, 4096, 2048, torch.float16, torch.float32, 0),     # fp16 x, fp32 scales
    (4, 512, 8192, torch.bfloat16, torch.float16, 0),     # 4 chunks per lane
    (4, 256, 16384, torch.bfloat16, torch.float16, 0),    # x too long for LDS: skinny kernel
    (8, 4095, 4096, torch.bfloat16, torch.float16, 128),  # INT8, ragged N, strided x
    (8, 2048, 8192, torch.float16, torch.float32, 0),     # INT8, 8 chunks per lane
])
def test_gemv_two_rows(dev, bits, N, K, dtype, sdt, pad):
    """M = 2 on the M = 1 GEMV's layout: both rows of x in LDS (row stride from the view),
    each weight chunk widened once for both rows; shapes it does not take fall back."""
    a, w = _data(2, N, K + pad, 300 + bits + N, 0.02)
    a = a.to(dtype)
    ax = a.to(dev)[:, :K] if pad else a.to(dev)
    w = w[:, :K].contiguous()
    if bits == 4:
        p, s = quantize_int4(w.to(dev), 128)
        s = s.to(sdt)
        out = int4_matmul(ax, p, s, 128)
        want = ref.int4_matmul(a[:, :K].float().numpy(), p.cpu().numpy(), s.float().cpu().numpy(), 128)
    else:
        q, s = quantize_int8(w.to(dev))
        s = s.to(sdt)
        out = int8_matmul(ax, q, s)
        want = ref.int8_matmul(a[:, :K].float().numpy(), q.cpu().numpy(), s.float().cpu().numpy())
    assert out.dtype == dtype and out.shape == (2, N)
    _check(out, want, f"two rows int{bits} N={N} K={K}")


@pytest.mark.parametrize("bits", [4, 8])
def test_gemv_two_rows_output_stride(dev, bits):
    """M = 2 through the C ABI into a wider output buffer: row 1 lands ldc elements after
    row 0, and the columns past N stay untouched."""
    import kernels
    from kernels._hip import stream
    M, N, K, pad = 2, 1000, 4096, 40
    a, w = _data(M, N, K, 400 + bits, 0.02)
    ab = a.to(torch.bfloat16).to(dev)
    c = torch.full((M, N + pad), 7.0, dtype=torch.bfloat16, device=dev)
    L = kernels.lib()
    if bits == 4:
        p, s = quantize_int4(w.to(dev), 128)
        s = s.to(torch.float16).contiguous()
        rc = L.mls_int4_gemm(ab.data_ptr(), kernels.MLS_BF16, K, p.data_ptr(), p.stride(0), s.data_ptr(),
                             kernels.MLS_F16, s.stride(0), 1, 128, c.data_ptr(), kernels.MLS_BF16, N + pad,
                             M, N, K, stream(dev))
        want = ref.int4_matmul(ab.float().cpu().numpy(), p.cpu().numpy(), s.float().cpu().numpy(), 128)
    else:
        q, s = quantize_int8(w.to(dev))
        s = s.to(torch.float16).contiguous()
        rc = L.mls_int8_gemm(ab.data_ptr(), kernels.MLS_BF16, K, q.data_ptr(), q.stride(0), s.data_ptr(),
                             kernels.MLS_F16, c.data_ptr(), kernels.MLS_BF16, N + pad, M, N, K, stream(dev))
        want = ref.int8_matmul(ab.float().cpu().numpy(), q.cpu().numpy(), s.float().cpu().numpy())
    torch.cuda.synchronize(dev)
    assert rc == 0
    _check(c[:, :N], want, f"two rows int{bits}, ldc = N + {pad}")
    assert torch.all(c[:, N:] == 7.0)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_int8_gemv_target(dev, M):
    """North-star INT8 GEMV: M=1, K = N = 4096, bf16 x, fp16 per-row scales."""
    a, w = _data(M, 4096, 4096, 200 + M, 0.02)
    q, s = quantize_int8(w.to(dev))
    s16 = s.to(torch.float16)
    ab = a.to(torch.bfloat16)
    out = int8_matmul(ab.to(dev), q, s16)
    _check(out, ref.int8_matmul(ab.float().numpy(), q.cpu().numpy(), s16.float().cpu().numpy()),
           f"int8 gemv M={M}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_gemv_other_dtypes(dev, dtype, M):
    a, p, s, want = _int4_setup(dev, M, 1024, 2048, 64, 300 + M, dtype)
    _check(int4_matmul(a, p, s, 64), want, f"int4 {dtype} M={M}")
    a2, w = _data(M, 768, 1536, 400 + M, 0.02)
    q, s8 = quantize_int8(w.to(dev))
    a2 = a2.to(dtype)
    _check(int8_matmul(a2.to(dev), q, s8),
           ref.int8_matmul(a2.float().numpy(), q.cpu().numpy(), s8.cpu().numpy()), f"int8 {dtype} M={M}")


@pytest.mark.parametrize("N,K,gs,sdt", [
    (4096, 4096, 128, torch.float16),  # the engine's decode shape: 4 rows per wavefront, 2 chunks per lane
    (1000, 3072, 32, torch.float16),   # ragged N, chunks past K
    (8200, 2048, 64, torch.float32),   # one chunk per lane, 8 rows per wavefront, fp32 scales, ragged block
    (300, 8192, 128, torch.float16),   # 4 chunks per lane: 32 KiB of fp32 x in LDS
    (77, 1088, 64, torch.float32),     # 34 chunks: most lanes past K
])
def test_gemv_m1_fp32_split(dev, N, K, gs, sdt):
    """INT4 M = 1 with fp32 x (the reference engine's decode dtype): x staged in LDS as fp32 and
    split into bf16 hi + lo parts, each dotted with the same widened weights; fp32 output within
    the fp32 rule of the oracle, with weights and scales as views with padded rows."""
    a, w = _data(1, N, K, 1300 + N, 0.02)
    p, s = quantize_int4(w.to(dev), gs)
    s = s.to(sdt)
    pw = torch.zeros(N, K // 2 + 32, dtype=torch.uint8, device=dev)
    pw[:, :K // 2] = p
    sw = torch.zeros(N, K // gs + 2, dtype=sdt, device=dev)
    sw[:, :K // gs] = s
    x = (a * torch.logspace(-3, 3, K)).float()  # magnitudes over six decades: the lo part matters
    out = int4_matmul(x.to(dev), pw[:, :K // 2], sw[:, :K // gs], gs)
    assert out.dtype == torch.float32
    _check(out, ref.int4_matmul(x.numpy(), p.cpu().numpy(), s.float().cpu().numpy(), gs),
           f"int4 fp32 M=1 N={N} K={K} g{gs}")


@pytest.mark.parametrize("N,K,gs,dtype,sdt", [
    (1000, 3072, 32, torch.bfloat16, torch.float16),   # ragged N, chunks past K, 4 scale instructions
    (777, 4096, 128, torch.float16, torch.float32),    # fp32 scales: 2 scale instructions per wavefront
    (64, 512, 128, torch.bfloat16, torch.float16),     # one chunk per lane; N < 8192: 2 rows per wavefront
    (4100, 2048, 64, torch.bfloat16, torch.float16),   # 2 rows per wavefront; last block holds 4 of its 8 rows
    (8200, 2048, 64, torch.bfloat16, torch.float16),   # N >= 8192: 8 rows per wavefront, last block ragged
])
def test_gemv_m1_edges(dev, N, K, gs, dtype, sdt):
    """M = 1 with 16-bit activations (x and scales through LDS): ragged N, K not a multiple of the
    lanes' span, both scale dtypes and slice sizes, weights and scales as views with padded rows."""
    a, w = _data(1, N, K, 900 + N, 0.02)
    p, s = quantize_int4(w.to(dev), gs)
    s = s.to(sdt)
    pw = torch.zeros(N, K // 2 + 48, dtype=torch.uint8, device=dev)   # ldw = K/2 + 48
    pw[:, :K // 2] = p
    sw = torch.zeros(N, K // gs + 6, dtype=sdt, device=dev)            # ld_sn = G + 6
    sw[:, :K // gs] = s
    ab = a.to(dtype)
    want = ref.int4_matmul(ab.float().numpy(), p.cpu().numpy(), s.float().cpu().numpy(), gs)
    _check(int4_matmul(ab.to(dev), pw[:, :K // 2], sw[:, :K // gs], gs), want, f"int4 M=1 N={N} K={K} g{gs}")
    q, s8 = quantize_int8(w.to(dev))
    s8 = s8.to(sdt)
    _check(int8_matmul(ab.to(dev), q, s8),
           ref.int8_matmul(ab.float().numpy(), q.cpu().numpy(), s8.float().cpu().numpy()), f"int8 M=1 N={N} K={K}")


def _scale_layout(s: torch.Tensor, layout: str) -> torch.Tensor:
    """The same [N, G] scale values under another stride pattern."""
    N, G = s.shape
    if layout == "transposed":        # stored [G][N]: strides (1, N)
        return s.t().contiguous().t()
    if layout == "row_broadcast":     # one row for every n: strides (0, 1)
        return s[:1].expand(N, G)
    if layout == "group_broadcast":   # one group for every k: strides (ld, 0)
        return s[:, :1].expand(N, G)
    if layout == "padded":            # rows G + 3 apart
        w = torch.zeros(N, G + 3, dtype=s.dtype, device=s.device)
        w[:, :G] = s
        return w[:, :G]
    raise ValueError(layout)


@pytest.mark.parametrize("layout", ["transposed", "row_broadcast", "group_broadcast", "padded"])
@pytest.mark.parametrize("M,N,K,gs,sdt", [
    (1, 1000, 4096, 128, torch.float16),    # M = 1 GEMV (x and scales through LDS where the strides allow)
    (2, 1000, 4096, 128, torch.float16),    # two-row GEMV / skinny kernel
    (4, 1000, 4096, 128, torch.float16),    # skinny MFMA kernel, scale slice in LDS
    (5, 1000, 1088, 64, torch.float32),     # skinny, 64-k steps, fp32 scales
    (64, 1000, 4096, 128, torch.float16),   # medium GEMM, scale table in LDS
    (300, 1000, 1024, 128, torch.float16),  # MFMA engine
])
def test_int4_scale_strides(dev, layout, M, N, K, gs, sdt):
    """int4_matmul honours any scale strides, as the reference does (dequant_matmul.py:182):
    transposed [G][N] storage, broadcast views with a zero stride and padded rows give the
    result of the same values stored contiguously."""
    a, w = _data(M, N, K, 1300 + M + N, 0.02)
    p, s = quantize_int4(w.to(dev), gs)
    sv = _scale_layout(s.to(sdt), layout)
    ab = a.to(torch.bfloat16)
    want = ref.int4_matmul(ab.float().numpy(), p.cpu().numpy(), sv.float().contiguous().cpu().numpy(), gs)
    _check(int4_matmul(ab.to(dev), p, sv, gs), want, f"int4 scales {layout} M={M} N={N} K={K} g{gs}")


def test_gemv_m1_unaligned_output_and_long_rows(dev):
    """Through the C ABI: an output that starts 2 bytes past an 8-byte boundary (element-wise
    stores), and K = 20480 (x beyond the LDS path: the register GEMV takes it)."""
    import kernels
    L = kernels.lib()
    st = torch.cuda.current_stream(dev).cuda_stream
    for N, K in ((300, 4096), (256, 20480)):
        a, p, s, want = _int4_setup(dev, 1, N, K, 128, 950 + K)
        buf = torch.full((N + 4,), float("nan"), dtype=torch.bfloat16, device=dev)
        out = buf[1:N + 1]
        rc = L.mls_int4_gemm(a.data_ptr(), kernels.MLS_BF16, K, p.data_ptr(), p.stride(0), s.data_ptr(),
                             kernels.MLS_F16, s.stride(0), 1, 128, out.data_ptr(), kernels.MLS_BF16, N, 1, N, K, st)
        assert rc == 0
        _check(out.reshape(1, N), want, f"int4 M=1 unaligned output N={N} K={K}")
        assert torch.isnan(buf[0]) and torch.isnan(buf[N + 1:]).all()


def test_gemv_long_k(dev):
    """K = 11008 (the down-projection's input): chunks do not divide evenly across lanes."""
    a, p, s, want = _int4_setup(dev, 1, 4096, 11008, 128, 7)
    _check(int4_matmul(a, p, s, 128), want, "int4 K=11008")
    a2, w = _data(2, 512, 11008, 8, 0.02)
    q, s8 = quantize_int8(w.to(dev))
    a2 = a2.to(torch.bfloat16)
    _check(int8_matmul(a2.to(dev), q, s8),
           ref.int8_matmul(a2.float().numpy(), q.cpu().numpy(), s8.cpu().numpy()), "int8 K=11008")


# --------------------------------------------------------------- skinny MFMA path (2 <= M <= 16)

@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (2, 4096, 4096, 128, torch.bfloat16),     # config B shape
    (16, 1000, 1152, 128, torch.bfloat16),    # N not a multiple of 16; 9 steps over 4 wavefronts
    (7, 333, 768, 256, torch.float16),        # group of two steps, odd M, ragged N
    (16, 4096, 14336, 128, torch.bfloat16),   # 112 steps: 16 wavefronts, chunks with tails
    (3, 48, 128, 128, torch.bfloat16),        # a single step: three wavefronts have none
    (16, 2048, 2048, 64, torch.float16),      # group 64: steps of 64 k (the reference's bench shape)
    (5, 1000, 1088, 64, torch.bfloat16),      # group 64, 17 steps, ragged N
    (9, 520, 576, 192, torch.float16),        # group 192: 64-k steps, a group spans three
])
def test_skinny_int4(dev, M, N, K, gs, dtype):
    a, p, s, want = _int4_setup(dev, M, N, K, gs, 500 + M, dtype)
    _check(int4_matmul(a, p, s, gs), want, f"skinny int4 M={M} N={N} K={K} g{gs}")


def test_skinny_int4_f32_scales_strided_rows(dev):
    M, N, K, gs = 5, 512, 1024, 128
    a, w = _data(M, N, K, 600, 0.02)
    p, s = quantize_int4(w.to(dev), gs)  # fp32 scales
    wide = torch.zeros(M, K + 64, dtype=torch.bfloat16)
    wide[:, :K] = a.to(torch.bfloat16)
    x = wide.to(dev)[:, :K]  # lda = K + 64
    want = ref.int4_matmul(wide[:, :K].float().numpy(), p.cpu().numpy(), s.cpu().numpy(), gs)
    _check(int4_matmul(x, p, s, gs), want, "skinny int4 fp32 scales, strided rows")


@pytest.mark.parametrize("M,N,K,dtype", [
    (2, 4096, 4096, torch.bfloat16),
    (16, 1000, 1088, torch.float16),   # 17 steps of 64 k
    (9, 77, 64, torch.bfloat16),       # one step, ragged N
    (16, 512, 14336, torch.bfloat16),  # 224 steps: 16 wavefronts, two chunks each
])
def test_skinny_int8(dev, M, N, K, dtype):
    a, w = _data(M, N, K, 700 + M, 0.02)
    q, s = quantize_int8(w.to(dev))
    s16 = s.to(torch.float16)
    ax = a.to(dtype)
    _check(int8_matmul(ax.to(dev), q, s16),
           ref.int8_matmul(ax.float().numpy(), q.cpu().numpy(), s16.float().cpu().numpy()),
           f"skinny int8 M={M} N={N} K={K}")


# --------------------------------------------------------------- medium path (16 < M <= 256, few tiles)

@pytest.mark.parametrize("M,N,K,dtype", [
    (128, 2048, 2048, torch.float16),    # reference bench shape
    (17, 1000, 1088, torch.bfloat16),    # one row past a tile, ragged N, 17 steps over 4 wavefronts
    (100, 333, 64, torch.bfloat16),      # a single step, odd N
    (250, 4096, 4096, torch.float16),    # near the top of the range: 4 x 4 tiles
])
def test_medium_int8(dev, M, N, K, dtype):
    a, w = _data(M, N, K, 800 + M, 0.02)
    q, s = quantize_int8(w.to(dev))
    s16 = s.to(torch.float16)
    ax = a.to(dtype)
    _check(int8_matmul(ax.to(dev), q, s16),
           ref.int8_matmul(ax.float().numpy(), q.cpu().numpy(), s16.float().cpu().numpy()),
           f"medium int8 M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (128, 2048, 2048, 128, torch.float16),
    (40, 1000, 1152, 128, torch.bfloat16),   # 9 steps: wavefronts of 2 and 3 steps
    (200, 520, 768, 256, torch.float16),     # a group spans two steps
    (33, 4096, 4096, 128, torch.bfloat16),
    (128, 2048, 2048, 64, torch.float16),    # group 64: steps of 64 k (the reference's bench shape)
    (40, 1000, 1088, 64, torch.bfloat16),    # group 64, 17 steps: wavefronts of 4 and 5 steps
    (130, 520, 576, 192, torch.float16),     # group 192: 64-k steps, a group spans three
])
def test_medium_int4(dev, M, N, K, gs, dtype):
    a, p, s, want = _int4_setup(dev, M, N, K, gs, 900 + M, dtype)
    _check(int4_matmul(a, p, s, gs), want, f"medium int4 M={M} N={N} K={K} g{gs}")


def test_medium_f32_scales_strided_rows(dev):
    M, N, K, gs = 70, 640, 1024, 128
    a, w = _data(M, N, K, 950, 0.02)
    p, s = quantize_int4(w.to(dev), gs)  # fp32 scales
    wide = torch.zeros(M, K + 64, dtype=torch.bfloat16)
    wide[:, :K] = a.to(torch.bfloat16)
    x = wide.to(dev)[:, :K]  # lda = K + 64
    want = ref.int4_matmul(wide[:, :K].float().numpy(), p.cpu().numpy(), s.cpu().numpy(), gs)
    _check(int4_matmul(x, p, s, gs), want, "medium int4 fp32 scales, strided rows")
    q, s8 = quantize_int8(w.to(dev))  # fp32 row scales
    _check(int8_matmul(x, q, s8), ref.int8_matmul(wide[:, :K].float().numpy(), q.cpu().numpy(),
                                                  s8.cpu().numpy()), "medium int8 fp32 scales")


# --------------------------------------------------------------- prefill (MFMA) path

@pytest.mark.parametrize("M,N,K", [(17, 256, 256), (64, 512, 512), (100, 300, 320),
                                   (256, 1024, 1024), (513, 768, 640)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mfma_int8(dev, M, N, K, dtype):
    a, w = _data(M, N, K, M + N + K, 0.02)
    q, s = quantize_int8(w.to(dev))
    a = a.to(dtype)
    out = int8_matmul(a.to(dev), q, s)
    _check(out, ref.int8_matmul(a.float().numpy(), q.cpu().numpy(), s.cpu().numpy()), f"int8 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [
    (1000, 11000, 512),   # 256 x 192 tiles, M and N ragged
    (4000, 4000, 256),    # 256 x 256 tiles (two rounds of 192-wide ones would be slower), ragged
    (2800, 8192, 256),    # 11 row tiles: runs of 4, 4 and 3 in the tile order
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mfma_int8_256_row_tiles(dev, M, N, K, dtype):
    """Shapes that take the 256-row INT8 kernel (widening interleaved with the MFMAs), with
    partial row and column tiles."""
    a, w = _data(M, N, K, M + N + K + 7, 0.02)
    q, s = quantize_int8(w.to(dev))
    a = a.to(dtype)
    out = int8_matmul(a.to(dev), q, s)
    _check(out, ref.int8_matmul(a.float().numpy(), q.cpu().numpy(), s.cpu().numpy()), f"int8 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,gs", [(17, 256, 256, 128), (64, 512, 512, 32), (100, 300, 320, 64),
                                      (256, 1024, 1024, 128), (513, 768, 640, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mfma_int4(dev, M, N, K, gs, dtype):
    a, p, s, want = _int4_setup(dev, M, N, K, gs, M + N + K + gs, dtype)
    _check(int4_matmul(a, p, s, gs), want, f"int4 {M}x{N}x{K} g{gs}")


@pytest.mark.parametrize("M,N,K,gs,dtype,sdt", [
    (1000, 3000, 4096, 128, torch.bfloat16, torch.float16),  # 256 x 128 tiles, M and N ragged, 32 groups
    (700, 520, 8192, 128, torch.bfloat16, torch.float16),    # 64 groups: the coefficient table's limit
    (512, 1024, 2048, 32, torch.bfloat16, torch.float16),    # groups of 32: a group end every k-step
    (600, 640, 1024, 64, torch.float16, torch.float32),      # fp16 x, fp32 scales, groups of 64
    (300, 256, 16384, 128, torch.bfloat16, torch.float16),   # 128 groups: the 128-row kernel instead
])
def test_mfma_int4_256_row_tiles(dev, M, N, K, gs, dtype, sdt):
    """Shapes that take the 256-row INT4 kernel (widening interleaved with the MFMAs, group
    scales by summation by parts from a coefficient table in LDS), with partial tiles."""
    a, w = _data(M, N, K, M + N + K + gs + 11, 0.02)
    p, s = quantize_int4(w.to(dev), gs)
    s = s.to(sdt)
    a = a.to(dtype)
    want = ref.int4_matmul(a.float().numpy(), p.cpu().numpy(), s.float().cpu().numpy(), gs)
    _check(int4_matmul(a.to(dev), p, s, gs), want, f"int4 {M}x{N}x{K} g{gs}")


def test_config_c_int8_prefill(dev):
    """INT8, x bf16 [2048, 4096], W [11008, 4096], fp16 scales, bf16 out."""
    M, N, K = 2048, 11008, 4096
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    q, s = quantize_int8(w)
    s16 = s.to(torch.float16)
    del w
    out = int8_matmul(a, q, s16)
    wd = q.float() * s16.float()[:, None]
    want = a.float() @ wd.t().contiguous()
    o = out.float()
    err = (o - want).abs() - (1e-2 + 1e-2 * want.abs())
    assert float(err.max()) <= 0, f"config C worst excess {float(err.max()):.3g}"
    rows = [0, 1, 777, 2047]
    _check(out[rows], ref.int8_matmul(a[rows].float().cpu().numpy(), q.cpu().numpy(),
                                      s16.float().cpu().numpy()), "config C rows")


def test_strided_activation(dev):
    a, w = _data(40, 256, 512, 5, 0.02)
    q, s = quantize_int8(w.to(dev))
    big = torch.zeros(40, 1024, dtype=torch.bfloat16, device=dev)
    big[:, 256:768] = a.to(torch.bfloat16).to(dev)
    view = big[:, 256:768]                         # row stride 1024
    out = int8_matmul(view, q, s)
    _check(out, ref.int8_matmul(a.bfloat16().float().numpy(), q.cpu().numpy(), s.cpu().numpy()), "strided")


def test_empty_m(dev):
    q, s = quantize_int8(torch.randn(16, 64, device=dev))
    out = int8_matmul(torch.zeros(0, 64, device=dev), q, s)
    assert out.shape == (0, 16)


# --------------------------------------------------------------- INT8 dgrad

# the reference rounds dy * s to dy's dtype before the dot (dequant_matmul.py:128)
_PRODUCT = {torch.float32: None, torch.bfloat16: "bf16", torch.float16: "fp16"}


@pytest.mark.parametrize("M,N,K", [(9, 24, 32), (33, 256, 512), (130, 300, 70), (300, 1000, 520)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_int8_dgrad(dev, M, N, K, dtype):
    g = torch.Generator().manual_seed(M + N)
    dy = torch.randn(M, N, generator=g).to(dtype)
    q, s = quantize_int8(torch.randn(N, K, generator=g))
    out = int8_dgrad(dy.to(dev), q.to(dev), s.to(dev))
    assert out.dtype == dtype and out.shape == (M, K)
    _check(out, ref.int8_dgrad(dy.float().numpy(), q.numpy(), s.numpy(), _PRODUCT[dtype]),
           f"dgrad {M}x{N}x{K}")


def test_int8_dgrad_training_shape(dev):
    """The STE backward at a training shape: dy [4096, 11008] bf16 x W_q [11008, 4096] on the
    matrix cores. Every output against torch fp32 of the reference's product on the GPU
    ((dy * s) rounded to bf16, times W_q, fp32 accumulation), within the bf16 tolerance
    |d| <= 1e-2 + 1e-2 |ref|; sampled rows against the CPU oracle."""
    M, N, K = 4096, 11008, 4096
    g = torch.Generator(device=dev).manual_seed(7)
    dy = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
    out = int8_dgrad(dy, q, s)
    assert out.dtype == torch.bfloat16 and out.shape == (M, K)
    want = (dy.float() * s.float()[None, :]).to(torch.bfloat16).float() @ q.float()
    err = (out.float() - want).abs() - (1e-2 + 1e-2 * want.abs())
    assert float(err.max()) <= 0, f"dgrad training shape: worst excess {float(err.max()):.3g}"
    rows = [0, 1, 2049, 4095]
    _check(out[rows], ref.int8_dgrad(dy[rows].float().cpu().numpy(), q.cpu().numpy(), s.cpu().numpy(), "bf16"),
           "dgrad training shape rows")


def test_int8_dgrad_strided_and_f16_scales(dev):
    M, N, K = 70, 192, 256
    g = torch.Generator().manual_seed(11)
    wide = torch.randn(M, N + 40, generator=g).to(torch.bfloat16)
    q, s = quantize_int8(torch.randn(N, K, generator=g))
    s16 = s.to(torch.float16)
    dyv = wide.to(dev)[:, 8:8 + N]  # row stride N + 40, offset 16 bytes
    out = int8_dgrad(dyv, q.to(dev), s16.to(dev))
    _check(out, ref.int8_dgrad(wide[:, 8:8 + N].float().numpy(), q.numpy(), s16.float().numpy(), "bf16"),
           "dgrad strided dy, fp16 scales")
