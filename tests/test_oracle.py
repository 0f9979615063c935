"""Pins the CPU oracle (oracle/ref.py) before it is trusted as the checker.

Each oracle function is checked against (a) the golden fixtures written by
tests/golden/make_golden.py from torch's CPU ops in the reference's order,
(b) torch live, where torch is the library the reference computes with, and
(c) what the mathematics fixes: brute-force loops on tiny inputs, round-trip
bounds and closed-form special cases. Planted mistakes in a copy of the oracle
must fail these checks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import ref


# ------------------------------------------------------------------ e4m3 decode


def test_decode_kat_all_256_patterns():
    """test_fp8.py:16-26: every byte equals torch's float8_e4m3fn view; the two NaN
    patterns 0x7F / 0xFF decode to 0 in the kernel semantics."""
    d = golden("e4m3_decode_kat")
    nan = np.isnan(d["value"])
    assert nan.sum() == 2 and set(np.nonzero(nan)[0]) == {0x7F, 0xFF}
    dec = ref.e4m3_decode(d["bits"])
    assert np.array_equal(dec[~nan].view(np.uint32), d["value"][~nan].view(np.uint32))
    assert (dec[nan] == 0).all()
    assert np.array_equal(ref.e4m3_decode(d["bits"], nan_to_zero=False), d["value"], equal_nan=True)
    live = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(live, d["value"], equal_nan=True)


def test_decode_closed_form_points():
    assert ref.E4M3_TABLE[0x7E] == 448.0          # max finite
    assert ref.E4M3_TABLE[0x01] == 2.0 ** -9      # smallest subnormal
    assert ref.E4M3_TABLE[0x08] == 2.0 ** -6      # smallest normal
    assert ref.E4M3_TABLE[0x38] == 1.0
    assert ref.E4M3_TABLE[0xB8] == -1.0
    finite = ref.E4M3_TABLE[:127]
    assert (np.diff(finite) > 0).all()            # codes 0x00..0x7E are ordered


# ------------------------------------------------------------------ e4m3 encode


@pytest.mark.parametrize("part", ["boundary", "random"])
def test_encode_matches_golden(part):
    e = golden("e4m3_encode")
    q = ref.quantize_e4m3(e[f"x_{part}"], 1.0)
    assert np.array_equal(q, e[f"q_{part}"])


def test_encode_scaled_and_per_row_match_golden():
    e = golden("e4m3_encode")
    assert np.array_equal(ref.quantize_e4m3(e["x_scaled"], float(e["scale"])), e["q_scaled"])
    assert np.array_equal(ref.quantize_e4m3(e["x_rows"], e["s_rows"]), e["q_rows"])
    assert np.array_equal(ref.dequantize_e4m3(e["q_scaled"], float(e["scale"])), e["dq_scaled"])


def test_encode_matches_torch_cast_live():
    g = np.random.default_rng(7)
    bits = g.integers(0, 2 ** 32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = np.where(np.isfinite(x), x, np.float32(1.0))
    near = (g.standard_normal(500_000) * np.exp2(g.integers(-12, 10, 500_000))).astype(np.float32)
    for v in (x, near):
        t = torch.from_numpy(v).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(ref.e4m3_encode(v), t)


@pytest.mark.slow
def test_encode_matches_torch_cast_dense():
    """All fp32 patterns of every binade that maps into e4m3's range, subsampled
    by a stride coprime to the mantissa grid."""
    for e in range(110, 137):
        base = np.uint32(e << 23)
        m = np.arange(0, 1 << 23, 7, dtype=np.uint32)
        v = (base | m).view(np.float32)
        v = np.concatenate([v, -v])
        t = torch.from_numpy(v).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(ref.e4m3_encode(v), t), f"binade {e}"


def test_encode_special_values():
    v = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 448.0, 464.0, 1e30, 2.0 ** -10], np.float32)
    q = ref.e4m3_encode(v)
    assert list(q[:4]) == [0x00, 0x80, 0x7E, 0xFE]
    assert q[4] & 0x7F == 0x7F
    assert list(q[5:8]) == [0x7E, 0x7E, 0x7E]
    assert q[8] == 0x00                        # 2^-10 < half the smallest subnormal


# ------------------------------------------------------------------ INT8 / INT4 quantizers


def test_quantize_int8_matches_golden():
    d = golden("quant_int8")
    q, s = ref.quantize_int8(d["w"])
    assert np.array_equal(q, d["w_q"]) and np.array_equal(s.view(np.uint32), d["scale"].view(np.uint32))
    assert (q[3] == 0).all() and s[3] == np.float32(1e-8)


@pytest.mark.parametrize("gs", [16, 32, 64, 128])
def test_quantize_int4_matches_golden(gs):
    d = golden("quant_int4")
    p, s = ref.quantize_int4(d[f"w_g{gs}"], gs)
    assert np.array_equal(p, d[f"packed_g{gs}"])
    assert np.array_equal(s.view(np.uint32), d[f"scale_g{gs}"].view(np.uint32))
    assert (ref.unpack_int4(p)[2, :gs] == 8).all()  # all-zero group -> stored nibble 8


def test_quantizers_match_torch_live():
    g = torch.Generator().manual_seed(11)
    w = torch.randn(96, 384, generator=g) * 0.02
    scale = (w.abs().amax(dim=1) / 127.0).clamp(min=1e-8)
    wq = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
    q, s = ref.quantize_int8(w.numpy())
    assert np.array_equal(q, wq.numpy()) and np.array_equal(s, scale.numpy())
    gq = w.reshape(96, 3, 128)
    s4 = (gq.abs().amax(dim=2) / 7.0).clamp(min=1e-8)
    q4 = (torch.round(gq / s4[:, :, None]).clamp(-8, 7) + 8).reshape(96, 384).to(torch.uint8)
    p4 = (q4[:, 0::2] | (q4[:, 1::2] << 4))
    p, s = ref.quantize_int4(w.numpy(), 128)
    assert np.array_equal(p, p4.numpy()) and np.array_equal(s, s4.numpy())


def test_roundtrip_error_bounded():
    """test_quantize.py:16-28: |w - dequant(quant(w))| <= scale / 2."""
    g = np.random.default_rng(0)
    w = g.standard_normal((64, 48)).astype(np.float32)
    q, s = ref.quantize_int8(w)
    assert (np.abs(w - ref.dequantize_int8(q, s)) <= s[:, None] / 2 + 1e-6).all()
    w = g.standard_normal((32, 64)).astype(np.float32)
    p, s = ref.quantize_int4(w, 16)
    bound = np.repeat(s, 16, axis=1) / 2 + 1e-6
    assert (np.abs(w - ref.dequantize_int4(p, s, 16)) <= bound).all()


def test_dequantize_int4_brute_force():
    g = np.random.default_rng(1)
    p = g.integers(0, 256, size=(3, 8), dtype=np.uint8)
    s = g.random((3, 4), dtype=np.float32) + 0.5
    w = ref.dequantize_int4(p, s, 4)
    for n in range(3):
        for k in range(16):
            byte = int(p[n, k // 2])
            nib = byte & 15 if k % 2 == 0 else byte >> 4
            assert w[n, k] == np.float32((nib - 8) * s[n, k // 4])


# ------------------------------------------------------------------ GEMM oracles


def _brute(a, w):
    M, K = a.shape
    N = w.shape[0]
    y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            y[m, n] = sum(float(a[m, k]) * float(w[n, k]) for k in range(K))
    return y


def test_int8_matmul_brute_force():
    g = np.random.default_rng(2)
    a = g.standard_normal((3, 7)).astype(np.float32)
    q = g.integers(-127, 128, size=(5, 7)).astype(np.int8)
    s = (g.random(5) + 0.1).astype(np.float32)
    y = ref.int8_matmul(a, q, s)
    yb = _brute(a, q.astype(np.float64)) * s[None, :]
    assert np.allclose(y, yb, rtol=1e-5, atol=1e-5)


def test_int4_matmul_brute_force():
    g = np.random.default_rng(3)
    a = g.standard_normal((2, 8)).astype(np.float32)
    p = g.integers(0, 256, size=(3, 4), dtype=np.uint8)
    s = (g.random((3, 2)) + 0.1).astype(np.float32)
    wd = np.zeros((3, 8))
    for n in range(3):
        for k in range(8):
            nib = (int(p[n, k // 2]) >> (4 * (k % 2))) & 15
            wd[n, k] = (nib - 8) * float(s[n, k // 4])
    assert np.allclose(ref.int4_matmul(a, p, s, 4), _brute(a, wd), rtol=1e-5, atol=1e-5)


def test_int8_dgrad_brute_force():
    g = np.random.default_rng(4)
    dy = g.standard_normal((3, 5)).astype(np.float32)
    q = g.integers(-127, 128, size=(5, 6)).astype(np.int8)
    s = (g.random(5) + 0.1).astype(np.float32)
    dx = np.zeros((3, 6))
    for m in range(3):
        for k in range(6):
            dx[m, k] = sum(float(dy[m, n]) * float(s[n]) * float(q[n, k]) for n in range(5))
    assert np.allclose(ref.int8_dgrad(dy, q, s), dx, rtol=1e-5, atol=1e-5)


def test_int8_dgrad_rounds_the_product_for_16bit_dy():
    """The reference rounds dy * s to dy's dtype before the dot (dequant_matmul.py:128).
    Known answers where that changes the result: bf16 (1 + 2^-7)(1 + 2^-8) = 1 + 1.5 2^-7
    + 2^-15 rounds up to 1 + 2^-6; fp16 (1 + 2^-10)(1 + 2^-11) rounds up to 1 + 2^-9. A
    planted omission of the rounding fails both."""
    one = np.ones((1, 1), dtype=np.int8)
    dy = np.array([[1 + 2.0 ** -7]], np.float32)
    s = np.array([1 + 2.0 ** -8], np.float32)
    assert ref.int8_dgrad(dy, one, s, "bf16")[0, 0] == np.float32(1 + 2.0 ** -6)
    assert ref.int8_dgrad(dy, one, s)[0, 0] == np.float32((1 + 2.0 ** -7) * (1 + 2.0 ** -8))
    dy = np.array([[1 + 2.0 ** -10]], np.float32)
    s = np.array([1 + 2.0 ** -11], np.float32)
    assert ref.int8_dgrad(dy, one, s, "fp16")[0, 0] == np.float32(1 + 2.0 ** -9)
    # rounding happens per product, before the sum: 4 products just above a tie
    q = np.ones((4, 1), dtype=np.int8)
    dy = np.full((1, 4), 1 + 2.0 ** -7, np.float32)
    s = np.full(4, 1 + 2.0 ** -8, np.float32)
    assert ref.int8_dgrad(dy, q, s, "bf16")[0, 0] == np.float32(4 * (1 + 2.0 ** -6))


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
def test_round_to_matches_torch_casts(dt):
    g = np.random.default_rng(9)
    x = np.concatenate([g.standard_normal(4096).astype(np.float32) * 10.0 ** g.integers(-6, 6, 4096),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3e38, -3e38, np.inf, -np.inf], np.float32)])
    # exact ties of the 16-bit grid: halfway points (round to even both ways)
    base = g.standard_normal(512).astype(np.float32)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    b16 = torch.from_numpy(base).to(tdt)
    nxt = torch.nextafter(b16.float().to(tdt).float(), torch.full_like(b16.float(), np.inf)).to(tdt)
    ties = ((b16.float() + nxt.float()) / 2).numpy()
    x = np.concatenate([x, ties]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = torch.from_numpy(x).to(tdt).float().numpy()
        got = ref.round_to(x, dt)
    assert np.array_equal(got, want, equal_nan=True)
    assert np.isnan(ref.round_to(np.array([np.nan], np.float32), dt)).all()


def test_fp8_matmul_brute_force_per_row_scales():
    g = np.random.default_rng(5)
    ab = g.integers(0, 256, size=(3, 9), dtype=np.uint8)
    bb = g.integers(0, 256, size=(4, 9), dtype=np.uint8)
    sa = (g.random(3) + 0.1).astype(np.float32)
    sb = (g.random(4) + 0.1).astype(np.float32)
    dec = lambda b: 0.0 if (b & 0x7F) == 0x7F else float(ref.E4M3_TABLE[b])  # noqa: E731
    y = np.zeros((3, 4))
    for m in range(3):
        for n in range(4):
            y[m, n] = sum(dec(ab[m, k]) * dec(bb[n, k]) for k in range(9)) * float(sa[m]) * float(sb[n])
    assert np.allclose(ref.fp8_matmul(ab, bb, sa, sb), y, rtol=1e-5, atol=1e-6)


def test_fp8_matmul_matches_golden():
    d = golden("fp8_small")
    for t in ("t1", "t2", "t3"):
        y = ref.fp8_matmul(d[f"{t}_a"], d[f"{t}_b"], float(d[f"{t}_sa"]), float(d[f"{t}_sb"]))
        assert np.allclose(y, d[f"{t}_y"], rtol=1e-5, atol=1e-5)


def test_int8_config_a_matches_golden():
    d = golden("gemm_int8_config_a")
    ok, worst = ref.close_fp32(ref.int8_matmul(d["x"], d["w_q"], d["scale"]), d["y"])
    assert ok and worst < 0.05


def test_int4_small_matches_golden():
    d = golden("gemm_int4_small")
    for t in ("t1", "t2", "t3", "g128"):
        y = ref.int4_matmul(d[f"{t}_a"], d[f"{t}_packed"], d[f"{t}_scale"], int(d[f"{t}_gs"]))
        assert np.allclose(y, d[f"{t}_y"], rtol=1e-5, atol=1e-5)


def test_grouped_matches_per_expert_loop():
    g = np.random.default_rng(6)
    E, N, K, gs = 3, 10, 64, 32
    p = g.integers(0, 256, size=(E, N, K // 2), dtype=np.uint8)
    s = (g.random((E, N, K // gs)) + 0.1).astype(np.float32)
    off = np.array([0, 4, 4, 9])
    a = g.standard_normal((9, K)).astype(np.float32)
    y = ref.grouped_int4_matmul(a, p, s, off, gs)
    assert np.allclose(y[:4], ref.int4_matmul(a[:4], p[0], s[0], gs))
    assert np.allclose(y[4:9], ref.int4_matmul(a[4:9], p[2], s[2], gs))


def test_silu_closed_forms_and_torch():
    x = np.linspace(-30, 30, 601)
    y = ref.silu(x)
    assert ref.silu(0.0) == 0.0
    assert np.allclose(y - ref.silu(-x), x, rtol=0, atol=1e-12)       # silu(x) - silu(-x) = x
    assert abs(ref.silu(40.0) - 40.0) < 1e-12 and abs(ref.silu(-40.0)) < 1e-12
    t = torch.nn.functional.silu(torch.from_numpy(x)).numpy()
    assert np.allclose(y, t, rtol=1e-12, atol=1e-15)


def test_gate_up_matches_per_row_formula():
    g = np.random.default_rng(7)
    E, H, K, gs = 3, 32, 64, 32
    wg = g.integers(0, 256, size=(E, H, K // 2), dtype=np.uint8)
    wu = g.integers(0, 256, size=(E, H, K // 2), dtype=np.uint8)
    sg = (g.random((E, H, K // gs)) * 0.05 + 0.01).astype(np.float32)
    su = (g.random((E, H, K // gs)) * 0.05 + 0.01).astype(np.float32)
    off = np.array([0, 3, 3, 8])
    a = g.standard_normal((8, K)).astype(np.float32)
    h = ref.grouped_int4_gate_up(a, wg, sg, wu, su, off, gs)
    for r in range(8):
        e = 0 if r < 3 else 2
        gate = ref.int4_matmul(a[r:r + 1], wg[e], sg[e], gs)[0].astype(np.float64)
        up = ref.int4_matmul(a[r:r + 1], wu[e], su[e], gs)[0].astype(np.float64)
        want = np.array([gv / (1 + np.exp(-gv)) * uv for gv, uv in zip(gate, up)])
        assert np.allclose(h[r], want, rtol=1e-5, atol=1e-5)
    # the down projection of the full MLP is the grouped GEMM of h
    D = 16
    wd = g.integers(0, 256, size=(E, D, H // 2), dtype=np.uint8)
    sd = (g.random((E, D, 1)) * 0.05).astype(np.float32)
    y = ref.grouped_int4_swiglu(a, wg, sg, wu, su, wd, sd, off, gs)
    assert np.allclose(y[3:], ref.int4_matmul(h[3:], wd[2], sd[2], gs), rtol=1e-5, atol=1e-5)


def test_combine_rows_pins():
    g = np.random.default_rng(8)
    T, K, D = 40, 2, 24
    x = g.standard_normal((T * K, D)).astype(np.float32)
    w = g.random((T, K)).astype(np.float32)
    pos = g.permutation(T * K).reshape(T, K)
    out = ref.combine_rows(x, w, pos)
    # the reference test's formula (test_moe_routing.py:21-28)
    assert np.allclose(out, (x[pos] * w[..., None]).sum(axis=1), rtol=1e-6, atol=1e-6)
    # brute force per element
    for t in (0, 17, 39):
        for d in (0, 23):
            assert abs(out[t, d] - sum(float(w[t, s]) * float(x[pos[t, s], d]) for s in range(K))) < 1e-9
    # one-hot weights: a gather; zero weights: zero; linear in the weights
    oh = np.zeros_like(w)
    oh[:, 1] = 1
    assert np.array_equal(ref.combine_rows(x, oh, pos), x[pos[:, 1]].astype(np.float64))
    assert not ref.combine_rows(x, np.zeros_like(w), pos).any()
    assert np.allclose(ref.combine_rows(x, 2 * w + oh, pos), 2 * out + x[pos[:, 1]], atol=1e-9)


def test_naive_route_equals_sorted_dispatch():
    g = np.random.default_rng(9)
    for T, E, k, D in [(64, 4, 2, 32), (37, 8, 1, 16), (16, 2, 2, 24)]:
        mats = g.standard_normal((E, D, D))
        fn = lambda e, rows: np.tanh(rows @ mats[e])  # noqa: E731
        flat = g.standard_normal((T, D))
        idx = g.integers(0, E, size=(T, k))
        if k == 2:
            idx[:, 1] = (idx[:, 0] + 1 + g.integers(0, E - 1, size=T)) % E
        w = g.random((T, k))
        w /= w.sum(-1, keepdims=True)
        tok, counts, pos = ref.sort_by_expert(idx, E)
        disp = flat[tok]
        eo = np.zeros_like(disp)
        off = np.concatenate([[0], np.cumsum(counts)])
        for e in range(E):
            eo[off[e]:off[e + 1]] = fn(e, disp[off[e]:off[e + 1]])
        assert np.allclose(ref.combine_rows(eo, w, pos), ref.naive_route(flat, w, idx, fn, E), atol=1e-12)
    # reference degenerate cases: every token to expert 0; zero weights
    flat = g.standard_normal((20, D))
    one = ref.naive_route(flat, np.ones((20, 1)), np.zeros((20, 1), np.int64), fn, 2)
    assert np.allclose(one, fn(0, flat))
    assert not ref.naive_route(flat, np.zeros((20, 2)), g.integers(0, 2, size=(20, 2)), fn, 2).any()


def _e5m2_boundaries():
    """Every midpoint between adjacent finite e5m2 values, one fp32 ulp either side,
    the values themselves, the clamp edge and the specials (both signs)."""
    v = ref._POS5_VALUES.astype(np.float64)
    mids = (v[:-1] + v[1:]) / 2
    pts = np.concatenate([v, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                          np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
                          [57344.0, 60000.0, 61439.0, 61440.0, 1e9, 2.0 ** -17, 3 * 2.0 ** -17, 2.0 ** -30]])
    pts = pts.astype(np.float32)
    return np.concatenate([pts, -pts, np.array([np.nan, -np.nan, np.inf, -np.inf], np.float32)])


def test_e5m2_decode_table_and_closed_forms():
    b = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(b).view(torch.float8_e5m2).float().numpy()
    assert np.array_equal(ref.e5m2_decode(b), t, equal_nan=True)
    d = ref.e5m2_decode(np.array([0x7B, 0x04, 0x01, 0x7C, 0xFC, 0x7D, 0x80], np.uint8))
    assert d[0] == 57344.0 and d[1] == 2.0 ** -14 and d[2] == 2.0 ** -16
    assert d[3] == np.inf and d[4] == -np.inf and np.isnan(d[5]) and d[6] == 0 and np.signbit(d[6])


@pytest.mark.parametrize("scale", [1.0, 0.37, 3e-6])
def test_quantize_e5m2_matches_torch_cast(scale):
    """train/fp8.py:50-52 run by torch on the CPU, on every rounding boundary (scaled
    back by the scale) and random samples."""
    g = np.random.default_rng(11)
    x = np.concatenate([_e5m2_boundaries() * np.float32(scale),
                        (g.standard_normal(20000) * 1e3 * scale).astype(np.float32)]).astype(np.float32)
    q = (torch.from_numpy(x).float() / scale).clamp(-57344.0, 57344.0)
    want = q.to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(ref.quantize_e5m2(x, scale), want)


def test_fp8_linear_backward_matches_torch_emulation():
    """The reference's backward op sequence (train/fp8.py:80-95) in torch fp64."""
    g = np.random.default_rng(12)
    M, N, K = 6, 5, 7
    dy = (g.standard_normal((M, N)) * 1e-3).astype(np.float32)
    xb = g.integers(0, 256, size=(M, K), dtype=np.uint8)
    wb = g.integers(0, 256, size=(N, K), dtype=np.uint8)
    xb[xb & 0x7F == 0x7F] = 0
    wb[wb & 0x7F == 0x7F] = 0
    sx, sw = 0.01, 0.002
    sdy = float(np.abs(dy).max()) / 57344.0
    dx, dw = ref.fp8_linear_backward(dy, xb, wb, sx, sw, sdy)
    q = (torch.from_numpy(dy) / sdy).clamp(-57344.0, 57344.0).to(torch.float8_e5m2)
    dyh = q.double() * torch.tensor(sdy, dtype=torch.float32).double()
    xh = torch.from_numpy(xb).view(torch.float8_e4m3fn).double() * np.float32(sx)
    wh = torch.from_numpy(wb).view(torch.float8_e4m3fn).double() * np.float32(sw)
    assert np.allclose(dx, (dyh @ wh).numpy(), rtol=1e-12, atol=0)
    assert np.allclose(dw, (dyh.t() @ xh).numpy(), rtol=1e-12, atol=0)
    # brute force for one element of each
    assert abs(dx[2, 3] - sum(float(dyh[2, n]) * float(wh[n, 3]) for n in range(N))) < 1e-15


def _scatter(ks, vs, H, D, bs, num_blocks, rng):
    """Write per-sequence contiguous K/V [H, L, D] into random free blocks of a pool;
    returns pools, padded tables and lengths."""
    kp = rng.standard_normal((num_blocks, H, bs, D))
    vp = rng.standard_normal((num_blocks, H, bs, D))
    free = list(rng.permutation(num_blocks))
    tables = []
    for k, v in zip(ks, vs):
        L = k.shape[1]
        blocks = [int(free.pop()) for _ in range((L + bs - 1) // bs)]
        for j in range(L):
            kp[blocks[j // bs], :, j % bs] = k[:, j]
            vp[blocks[j // bs], :, j % bs] = v[:, j]
        tables.append(blocks)
    mb = max(len(t) for t in tables)
    tab = np.array([t + [0] * (mb - len(t)) for t in tables], dtype=np.int32)
    return kp, vp, tab, np.array([k.shape[1] for k in ks], dtype=np.int32)


def test_attention_matches_torch_sdpa_and_closed_forms():
    g = np.random.default_rng(13)
    q, k, v = g.standard_normal(16), g.standard_normal((9, 16)), g.standard_normal((9, 16))
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[None, None], torch.from_numpy(k)[None], torch.from_numpy(v)[None])[0, 0]
    assert np.allclose(ref.attention(q, k, v, 16 ** -0.5), want.numpy(), rtol=1e-12, atol=1e-12)
    assert np.allclose(ref.attention(q, k[:1], v[:1], 0.3), v[0])
    assert np.allclose(ref.attention(q, np.repeat(k[:1], 5, 0), v[:5], 0.3), v[:5].mean(0))


@pytest.mark.parametrize("lens", [[7], [16], [5, 23, 12], [1, 1, 40]])
def test_paged_oracle_matches_contiguous(lens):
    """test_serving.py:62-84 of the reference, on the oracle: paged == contiguous."""
    g = np.random.default_rng(sum(lens))
    H, D, bs = 4, 32, 8
    ks = [g.standard_normal((H, L, D)) for L in lens]
    vs = [g.standard_normal((H, L, D)) for L in lens]
    kp, vp, tab, ctx = _scatter(ks, vs, H, D, bs, 32, g)
    q = g.standard_normal((len(lens), H, D))
    out = ref.paged_attention_decode(q, kp, vp, tab, ctx)
    for i in range(len(lens)):
        for h in range(H):
            assert np.allclose(out[i, h], ref.attention(q[i, h], ks[i][h], vs[i][h], D ** -0.5), atol=1e-12)
    # a permutation of the pool's blocks, with the tables renamed alike, changes nothing
    perm = g.permutation(32)
    inv = np.argsort(perm)
    out2 = ref.paged_attention_decode(q, kp[perm], vp[perm], inv[tab].astype(np.int32), ctx)
    assert np.allclose(out, out2, atol=1e-12)


def test_paged_oracle_ignores_slots_past_context():
    """test_serving.py:87-106: poisoned slots of a partially filled block do not leak."""
    g = np.random.default_rng(14)
    H, D, bs = 2, 16, 8
    k, v = g.standard_normal((1, H, 5, D)), g.standard_normal((1, H, 5, D))
    kp, vp, tab, ctx = _scatter([k[0]], [v[0]], H, D, bs, 4, g)
    kp[tab[0, 0], :, 5:] = 1e6
    vp[tab[0, 0], :, 5:] = 1e6
    q = g.standard_normal((1, H, D))
    out = ref.paged_attention_decode(q, kp, vp, tab, ctx)
    assert np.allclose(out[0, 1], ref.attention(q[0, 1], k[0, 1], v[0, 1], D ** -0.5), atol=1e-12)
    # planted: counting one token too many picks up the poison
    bad = ref.paged_attention_decode(q, kp, vp, tab, ctx + 1)
    assert not np.allclose(bad, out, atol=1e-3)


def test_routing_matches_golden():
    d = golden("route_small")
    w, ex = ref.route_topk(d["logits"], 2)
    assert np.array_equal(ex, d["experts"]) and np.allclose(w, d["weights"], rtol=1e-6, atol=1e-7)
    tok, counts, pos = ref.sort_by_expert(d["experts"], 8)
    assert np.array_equal(tok, d["token_of_slot"]) and np.array_equal(counts, d["counts"])
    assert np.array_equal(pos, d["pos"])


def test_tolerance_helpers():
    ref_ = np.array([1.0, -2.0, 0.0], np.float32)
    assert ref.close_bf16(ref_ + 0.009, ref_)[0] and not ref.close_bf16(ref_ + 0.05, ref_)[0]
    assert ref.close_fp32(ref_ * (1 + 2 ** -11), ref_)[0]
    assert not ref.close_fp32(ref_ * (1 + 2 ** -7), ref_)[0]


# ------------------------------------------------------------------ planted mistakes


def test_planted_mistakes_fail_the_pins():
    d = golden("quant_int4")
    w = d["w_g32"]
    # nibble order swapped (odd k in the low nibble)
    q = (np.clip(np.rint(w.reshape(32, 8, 32) / d["scale_g32"][:, :, None]), -8, 7) + 8)
    q = q.reshape(32, 256).astype(np.uint8)
    swapped = (q[:, 1::2] | (q[:, 0::2] << 4)).astype(np.uint8)
    assert not np.array_equal(swapped, d["packed_g32"])
    # offset 7 instead of 8 in the dequantizer changes the GEMM beyond tolerance
    gm = golden("gemm_int4_small")
    p, s, a = gm["g128_packed"], gm["g128_scale"], gm["g128_a"]
    wrong = ((ref.unpack_int4(p).astype(np.float32) - 7).reshape(40, 4, 128) * s[:, :, None]).reshape(40, 512)
    assert not ref.close_fp32(a @ wrong.T, gm["g128_y"])[0]
    # transposed operand / scale applied per column instead of per row
    da = golden("gemm_int8_config_a")
    bad = da["x"] @ (da["w_q"].astype(np.float32) * da["scale"][:8, None].mean()).T
    assert not ref.close_fp32(bad, da["y"])[0]
    # e4m3 rounding ties away from zero instead of to even
    e = golden("e4m3_encode")
    x = e["x_boundary"].astype(np.float64)
    a_ = np.minimum(np.abs(x), 448)
    hi = np.minimum(np.searchsorted(ref._POS_VALUES, a_), 126)
    lo = np.maximum(hi - 1, 0)
    away = np.where(ref._POS_VALUES[hi] - a_ <= a_ - ref._POS_VALUES[lo], hi, lo)
    finite = np.isfinite(x)
    assert not np.array_equal(away[finite].astype(np.uint8), e["q_boundary"][finite] & 0x7F)
    # gate and up swapped in the SwiGLU product
    g = np.random.default_rng(10)
    wg = g.integers(0, 256, size=(1, 8, 32), dtype=np.uint8)
    wu = g.integers(0, 256, size=(1, 8, 32), dtype=np.uint8)
    sc = np.full((1, 8, 2), 0.05, np.float32)
    a = g.standard_normal((4, 64)).astype(np.float32)
    off = np.array([0, 4])
    h = ref.grouped_int4_gate_up(a, wg, sc, wu, sc, off, 32)
    assert not ref.close_fp32(ref.grouped_int4_gate_up(a, wu, sc, wg, sc, off, 32), h)[0]
    # e5m2 ties rounded away from zero instead of to even
    v = ref._POS5_VALUES
    mids = ((v[:-1] + v[1:]) / 2).astype(np.float32)
    away = np.arange(1, len(v)).astype(np.uint8)              # always the upper neighbour
    assert not np.array_equal(away, ref.quantize_e5m2(mids, 1.0))
    # combine reading pos transposed ([k, T] order)
    x = g.standard_normal((12, 4))
    w = g.random((6, 2))
    pos = g.permutation(12).reshape(6, 2)
    assert not np.allclose(ref.combine_rows(x, w, pos.T.reshape(6, 2)), (x[pos] * w[..., None]).sum(1))


# ------------------------------------------------------------------ the reference's torch CPU path


def test_torch_cpu_path_matches_oracle():
    """oracle/torch_cpu.py (the op sequences bench.py's cpu_baseline times) against the
    numpy oracle: dequantizers bit for bit on the golden quantizer fixtures, the
    QuantLinear(use_kernel=False) linear and the FP8 emulation within the fp32 bound,
    the 16-bit linear after its weight rounding to x's dtype within the bf16 bound."""
    from oracle import torch_cpu as tc
    d8 = golden("quant_int8")
    wq8, s8 = torch.from_numpy(d8["w_q"]), torch.from_numpy(d8["scale"])
    assert np.array_equal(tc.dequantize_int8(wq8, s8).numpy(), ref.dequantize_int8(d8["w_q"], d8["scale"]))
    g = np.random.default_rng(21)
    for gs in (32, 128):
        w = (g.standard_normal((48, 256)) * 0.02).astype(np.float32)
        p, s = ref.quantize_int4(w, gs)
        got = tc.dequantize_int4(torch.from_numpy(p), torch.from_numpy(s), gs).numpy()
        assert np.array_equal(got, ref.dequantize_int4(p, s, gs))
        x = g.standard_normal((3, 256)).astype(np.float32)
        y = tc.quant_linear(torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(s), 4, gs).numpy()
        assert ref.close_fp32(y, ref.int4_matmul(x, p, s, gs))[0]
        yb = tc.quant_linear(torch.from_numpy(x).bfloat16(), torch.from_numpy(p), torch.from_numpy(s).half(), 4, gs)
        assert yb.dtype == torch.bfloat16
        assert ref.close_bf16(yb.float().numpy(), ref.int4_matmul(x, p, s.astype(np.float16), gs))[0]
    x = g.standard_normal((5, d8["w_q"].shape[1])).astype(np.float32)
    y = tc.quant_linear(torch.from_numpy(x), wq8, s8, 8).numpy()
    assert ref.close_fp32(y, ref.int8_matmul(x, d8["w_q"], d8["scale"]))[0]
    a, b = g.standard_normal((9, 64)).astype(np.float32), g.standard_normal((7, 64)).astype(np.float32)
    sa, sb = np.abs(a).max(1) / 448, np.abs(b).max(1) / 448
    ab, bb = ref.quantize_e4m3(a, sa[:, None]), ref.quantize_e4m3(b, sb[:, None])
    y = tc.fp8_linear_emulated(torch.from_numpy(ab), torch.from_numpy(bb), torch.from_numpy(sa)[:, None].float(),
                               torch.from_numpy(sb)[:, None].float()).numpy()
    assert ref.close_fp32(y, ref.fp8_matmul(ab, bb, sa, sb))[0]
    # a planted mistake: the nibbles unpacked high-first
    p, s = ref.quantize_int4((g.standard_normal((8, 64)) * 0.02).astype(np.float32), 32)
    swapped = ((p >> 4) | ((p & 0x0F) << 4)).astype(np.uint8)
    assert not np.array_equal(tc.dequantize_int4(torch.from_numpy(swapped), torch.from_numpy(s), 32).numpy(),
                              ref.dequantize_int4(p, s, 32))
