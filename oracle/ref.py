"""CPU oracle for the quantized-linear path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A numpy restatement of the reference's arithmetic for this path, used only by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker
(and, for the baseline, as the reference's CPU algorithm being timed). The
product (mini-llm-stack_amd/) never imports it.

Each function cites the reference code it restates. Pins (see tests/test_oracle.py):
  e4m3_decode      256-byte known-answer table of torch's float8_e4m3fn view
                   (test_fp8.py:16-26 of the reference) + golden fixture.
  e4m3_encode      torch's float8_e4m3fn cast on every rounding boundary, the
                   special values and random samples (golden fixture and live).
                   Implemented by nearest-value search over the 126 finite
                   magnitudes, not by bit manipulation, so that it is an
                   independent derivation from the HIP encoder.
  quantize_int8/4  torch op sequences of serve/quantize.py (golden fixtures),
                   round-trip bound |w - dq| <= s/2 (test_quantize.py:16-28),
                   all-zero rows/groups, exact ties.
  dequantize_*     closed form; brute-force per-element loop on tiny inputs.
  *_matmul         fp64 brute-force triple loop on tiny inputs; golden fixture
                   of config A produced by torch's fp32 matmul.
  int8_dgrad       fp64 brute force on tiny inputs; the rounding of dy * s for 16-bit
                   dy by known answers where it changes the result (1 + 2^-7 times
                   1 + 2^-8 is 1 + 2^-6 in bf16) and round_to against torch's bf16 /
                   fp16 casts on random values and ties.
  route / sort     torch softmax/topk/argsort golden fixture.
  silu             closed forms: silu(0) = 0, silu(x) - silu(-x) = x, silu(x) -> x
                   and -> 0 at the tails; torch.nn.functional.silu on the CPU.
  grouped_*        per-expert loop against int4_matmul on each segment; gate/up
                   against silu(int4_matmul) * int4_matmul computed per row.
  combine_rows     the reference test's formula (test_moe_routing.py:21-28), brute
                   force per element, one-hot weights reduce it to a gather, zero
                   weights to zero, linearity in the weights.
  e5m2_decode      torch's float8_e5m2 view of all 256 patterns (live) and closed-form
                   points (max 57344, min normal 2^-14, min subnormal 2^-16, inf, NaN).
  quantize_e5m2    torch's float8_e5m2 cast after the reference's clamp on every rounding
                   boundary and random samples (live torch).
  fp8_linear_backward  the reference's emulation sequence in torch fp64 on tiny inputs.
  attention        torch's scaled_dot_product_attention on the CPU; closed forms (one key
                   -> its value; equal keys -> the mean of the values).
  paged_attention_decode  equals attention() on the contiguous K/V it was scattered from
                   (the reference's test, test_serving.py:62-84); poisoned slots past the
                   context are ignored (:87-106); invariant under a permutation of the
                   pool's blocks with the tables permuted alike.
  naive_route      equals sort_by_expert + per-segment experts + combine_rows on
                   random routings (two formulations of the same forward), and the
                   reference's degenerate cases (all tokens to one expert,
                   test_moe_routing.py:64-82).
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0

# ------------------------------------------------------------------ e4m3 (OCP "fn")


def _e4m3_table() -> np.ndarray:
    """Value of every byte: 1 sign, 4 exponent bits (bias 7), 3 mantissa bits;
    exponent 0 is subnormal (m/8 * 2^-6); S.1111.111 is NaN; no infinities
    (kernels/fp8_matmul.py:20-21, 37-47)."""
    vals = np.empty(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 15 and m == 7:
            vals[b] = np.nan
        elif e == 0:
            vals[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


E4M3_TABLE = _e4m3_table()
_POS_CODES = np.arange(0, 127)                 # 0x00 .. 0x7E: finite non-negative values
_POS_VALUES = E4M3_TABLE[_POS_CODES]           # strictly increasing


def e4m3_decode(bits: np.ndarray, nan_to_zero: bool = True) -> np.ndarray:
    """fp32 values of e4m3 bytes. nan_to_zero follows the reference kernel's decode
    (kernels/fp8_matmul.py:46: the NaN patterns decode to a signed 0); False follows
    torch's float8 view (NaN stays NaN, kernels/fp8_matmul.py:110)."""
    bits = np.asarray(bits, dtype=np.uint8)
    v = E4M3_TABLE[bits]
    if nan_to_zero:
        nan = np.isnan(v)
        v = np.where(nan, np.where(bits & 0x80, -0.0, 0.0), v)
    return v.astype(np.float32)


def e4m3_encode(q: np.ndarray) -> np.ndarray:
    """e4m3 code of q (already divided by the scale): clamp to [-448, 448]
    (kernels/fp8_matmul.py:105), then the nearest representable value, ties to the
    even code (torch's float8_e4m3fn cast, :106). NaN -> 0x7F with q's sign bit."""
    q = np.asarray(q, dtype=np.float32)
    sign = (q.view(np.uint32) >> 31).astype(np.uint8) << 7
    a = np.minimum(np.abs(q.astype(np.float64)), E4M3_MAX)
    hi = np.searchsorted(_POS_VALUES, a, side="left")          # first value >= a
    hi = np.minimum(hi, len(_POS_VALUES) - 1)
    lo = np.maximum(hi - 1, 0)
    d_lo = a - _POS_VALUES[lo]
    d_hi = _POS_VALUES[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (_POS_CODES[hi] % 2 == 0))
    code = np.where(pick_hi, _POS_CODES[hi], _POS_CODES[lo]).astype(np.uint8)
    code = np.where(np.isnan(q), np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)


def quantize_e4m3(x: np.ndarray, scale) -> np.ndarray:
    """kernels/fp8_matmul.py:103-106 with IEEE fp32 division by float32(scale)
    (scale: a float or an array broadcastable against x)."""
    q = np.asarray(x, dtype=np.float32) / np.asarray(scale, dtype=np.float32)
    return e4m3_encode(q.astype(np.float32))


def dequantize_e4m3(bits: np.ndarray, scale) -> np.ndarray:
    """kernels/fp8_matmul.py:109-110: exact value times the scale, one fp32 rounding."""
    return (e4m3_decode(bits, nan_to_zero=False) * np.asarray(scale, dtype=np.float32)).astype(
        np.float32)


# ------------------------------------------------------------------ e5m2 (FP8 training gradients)

E5M2_MAX = 57344.0


def _e5m2_table() -> np.ndarray:
    """Value of every byte: 1 sign, 5 exponent bits (bias 15), 2 mantissa bits;
    exponent 0 is subnormal (m/4 * 2^-14); exponent 31 is inf (m = 0) or NaN
    (OCP E5M2, torch.float8_e5m2; train/fp8.py:50-56)."""
    vals = np.empty(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 2) & 0x1F
        m = b & 0x3
        if e == 31:
            vals[b] = s * np.inf if m == 0 else np.nan
        elif e == 0:
            vals[b] = s * (m / 4.0) * 2.0 ** -14
        else:
            vals[b] = s * (1.0 + m / 4.0) * 2.0 ** (e - 15)
    return vals


E5M2_TABLE = _e5m2_table()
_POS5_CODES = np.arange(0, 0x7C)               # 0x00 .. 0x7B: finite non-negative values
_POS5_VALUES = E5M2_TABLE[_POS5_CODES]


def e5m2_decode(bits: np.ndarray) -> np.ndarray:
    """fp32 values of e5m2 bytes (torch's float8_e5m2 view, train/fp8.py:55-56)."""
    return E5M2_TABLE[np.asarray(bits, dtype=np.uint8)].astype(np.float32)


def quantize_e5m2(x: np.ndarray, scale) -> np.ndarray:
    """train/fp8.py:50-52: q = float32(x) / float32(scale) (IEEE), clamp to
    ±57344, then the nearest e5m2 value, ties to the even code (torch's cast);
    NaN -> 0x7F with q's sign. Nearest-value search, like e4m3_encode."""
    q = (np.asarray(x, dtype=np.float32) / np.asarray(scale, dtype=np.float32)).astype(np.float32)
    sign = (q.view(np.uint32) >> 31).astype(np.uint8) << 7
    a = np.minimum(np.abs(q.astype(np.float64)), E5M2_MAX)
    hi = np.minimum(np.searchsorted(_POS5_VALUES, a, side="left"), len(_POS5_VALUES) - 1)
    lo = np.maximum(hi - 1, 0)
    d_lo, d_hi = a - _POS5_VALUES[lo], _POS5_VALUES[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (_POS5_CODES[hi] % 2 == 0))
    code = np.where(pick_hi, _POS5_CODES[hi], _POS5_CODES[lo]).astype(np.uint8)
    code = np.where(np.isnan(q), np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)


def fp8_linear_backward(dy, xb, wb, sx, sw, sdy):
    """_FP8LinearFn.backward (train/fp8.py:80-95) in fp64: dy re-quantized to e5m2
    with scale sdy, then dx = dyh @ wh and dw = dyh^T @ xh against the forward's e4m3
    operands xb [M,K] and wb [N,K] (scales sx, sw). Returns (dx [M,K], dw [N,K])."""
    dyh = e5m2_decode(quantize_e5m2(dy, sdy)).astype(np.float64) * np.float32(sdy)
    xh = E4M3_TABLE[np.asarray(xb, dtype=np.uint8)] * np.float32(sx)
    wh = E4M3_TABLE[np.asarray(wb, dtype=np.uint8)] * np.float32(sw)
    return dyh @ wh, dyh.T @ xh


# ------------------------------------------------------------------ INT8 / INT4 weights


def quantize_int8(w: np.ndarray):
    """serve/quantize.py:18-21."""
    w = np.asarray(w, dtype=np.float32)
    scale = np.maximum(np.abs(w).max(axis=1) / np.float32(127.0), np.float32(1e-8))
    q = np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale.astype(np.float32)


def dequantize_int8(w_q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """serve/quantize.py:24-25."""
    return (w_q.astype(np.float32) * np.asarray(scale, dtype=np.float32)[:, None]).astype(np.float32)


def quantize_int4(w: np.ndarray, group_size: int = 32):
    """serve/quantize.py:28-36: unsigned nibbles with offset 8, even k in the low nibble."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    assert K % group_size == 0
    g = w.reshape(N, K // group_size, group_size)
    scale = np.maximum(np.abs(g).max(axis=2) / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(g / scale[:, :, None]), -8, 7) + 8
    q = q.reshape(N, K).astype(np.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, scale


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Stored nibbles (0..15) [N, K] of packed [N, K/2]."""
    packed = np.asarray(packed, dtype=np.uint8)
    N, H = packed.shape
    q = np.empty((N, 2 * H), dtype=np.uint8)
    q[:, 0::2] = packed & 0x0F
    q[:, 1::2] = packed >> 4
    return q


def dequantize_int4(packed: np.ndarray, scale: np.ndarray, group_size: int) -> np.ndarray:
    """serve/quantize.py:39-47."""
    q = unpack_int4(packed).astype(np.float32) - np.float32(8.0)
    N, K = q.shape
    s = np.asarray(scale, dtype=np.float32)
    return (q.reshape(N, K // group_size, group_size) * s[:, :, None]).reshape(N, K).astype(np.float32)


# ------------------------------------------------------------------ GEMMs (dequantize, fp32 matmul)


def _f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def int8_matmul(a, w_q, scale) -> np.ndarray:
    """a @ dequantize_int8(w_q, s).T in fp32 (test_quantize.py:37; dequant_matmul.py:140-152)."""
    return (_f32(a) @ dequantize_int8(w_q, scale).T).astype(np.float32)


def int4_matmul(a, packed, scale, group_size) -> np.ndarray:
    """a @ dequantize_int4(...).T in fp32 (test_quantize.py:48; dequant_matmul.py:170-185)."""
    return (_f32(a) @ dequantize_int4(packed, scale, group_size).T).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 / fp16 (ties to even), returned as fp32.
    bf16: round the fp32 bit pattern at bit 16 (NaN kept); fp16: numpy's float16 cast."""
    x = _f32(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    assert dtype == "bf16", dtype
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return np.where(np.isnan(x), x, r.view(np.float32))


def int8_dgrad(dy, w_q, scale, product_dtype: str | None = None) -> np.ndarray:
    """(dy * s) @ w_q, fp32 accumulation (dequant_matmul.py:103-132; kaggle/gpu_smoke.py:
    133-135 for fp32 dy). The reference forms dy * s in fp32 and rounds it to dy's dtype
    before the dot ((dy * s[None, :]).to(dy.dtype), dequant_matmul.py:128): pass
    product_dtype "bf16" / "fp16" for 16-bit dy, None for fp32 dy (no rounding)."""
    ys = _f32(dy) * _f32(scale)[None, :]
    if product_dtype is not None:
        ys = round_to(ys, product_dtype)
    return (ys @ np.asarray(w_q).astype(np.float32)).astype(np.float32)


def fp8_matmul(a_bits, b_bits, sa, sb) -> np.ndarray:
    """(decode(A) @ decode(B).T) * (sa * sb), decode with NaN -> 0
    (kernels/fp8_matmul.py:50-81). sa / sb: floats or per-row arrays [M] / [N]."""
    acc = e4m3_decode(a_bits) @ e4m3_decode(b_bits).T
    sa = np.asarray(sa, dtype=np.float32).reshape(-1, 1) if np.ndim(sa) else np.float32(sa)
    sb = np.asarray(sb, dtype=np.float32).reshape(1, -1) if np.ndim(sb) else np.float32(sb)
    return (acc * (sa * sb)).astype(np.float32)


def grouped_int4_matmul(a_sorted, packed, scale, offsets, group_size) -> np.ndarray:
    """Per-expert segment loop of kernels/moe_routing.py:145-151 with int4 experts:
    rows offsets[e]:offsets[e+1] times expert e's dequantized weights."""
    a = _f32(a_sorted)
    E, N, _ = packed.shape
    out = np.zeros((a.shape[0], N), dtype=np.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            out[lo:hi] = a[lo:hi] @ dequantize_int4(packed[e], scale[e], group_size).T
    return out


def silu(x) -> np.ndarray:
    """x * sigmoid(x) in fp64 (torch.nn.functional.silu, train/model.py:135)."""
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def grouped_int4_gate_up(a_sorted, wg, sg, wu, su, offsets, group_size) -> np.ndarray:
    """silu(x Wg_e^T) * (x Wu_e^T) for every row of expert e's segment: the inner
    product of SwiGLU.forward (train/model.py:134-135) with INT4 gate/up experts, one
    rounding at the end (fp32 result)."""
    g = grouped_int4_matmul(a_sorted, wg, sg, offsets, group_size).astype(np.float64)
    u = grouped_int4_matmul(a_sorted, wu, su, offsets, group_size).astype(np.float64)
    return (silu(g) * u).astype(np.float32)


def grouped_int4_swiglu(a_sorted, wg, sg, wu, su, wd, sd, offsets, group_size) -> np.ndarray:
    """w_down(silu(w_gate(x)) * w_up(x)) per expert segment (train/model.py:134-135,
    kernels/moe_routing.py:145-151) with INT4 projections; the hidden activation h
    stays fp32 (a caller modelling a 16-bit h rounds it itself)."""
    h = grouped_int4_gate_up(a_sorted, wg, sg, wu, su, offsets, group_size)
    return grouped_int4_matmul(h, wd, sd, offsets, group_size)


def combine_rows(expert_out, weights, pos) -> np.ndarray:
    """kernels/moe_routing.py:52-76, 100-113: out[t] = sum_k weights[t, k] *
    expert_out[pos[t, k]], accumulated over k in order (fp64 here)."""
    x = np.asarray(expert_out, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    pos = np.asarray(pos)
    T, K = pos.shape
    out = np.zeros((T, x.shape[1]), dtype=np.float64)
    for s in range(K):
        out += w[:, s:s + 1] * x[pos[:, s]]
    return out


def naive_route(flat, weights, experts_idx, expert_fn, n_experts) -> np.ndarray:
    """train/model.py:178-187 (_naive_route): for each expert, the tokens routed to
    it, expert_fn(e, rows) scaled by their router weight, index-added into the output.
    No sort, no inverse permutation: an independent formulation of the routed MoE
    forward that moe_dispatch_combine (kernels/moe_routing.py:133-153) must equal."""
    x = np.asarray(flat, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    out = np.zeros_like(x)
    for e in range(n_experts):
        tok, slot = np.nonzero(np.asarray(experts_idx) == e)
        if tok.size:
            np.add.at(out, tok, np.asarray(expert_fn(e, x[tok]), dtype=np.float64) * w[tok, slot, None])
    return out


# ------------------------------------------------------------------ paged-attention decode


def attention(q, k, v, scale) -> np.ndarray:
    """softmax(scale * q k^T) v in fp64 for one query row (train/model.py:55-70 with
    causal=False: the decode case, every cached key visible). q [D], k, v [L, D]."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    if k.shape[0] == 0:
        return np.zeros(q.shape[-1])
    s = (k @ q) * scale
    p = np.exp(s - s.max())
    return (p / p.sum()) @ v


def paged_attention_decode(q, k_pool, v_pool, block_tables, context_lens, scale=None) -> np.ndarray:
    """kernels/paged_attention.py:33-118: for each (sequence, head), the keys and values
    of the sequence's first context_lens[s] tokens, token j at row j % block_size of
    block block_tables[s][j // block_size], attended by q[s, h]. fp64 result."""
    q = np.asarray(q)
    n, H, D = q.shape
    bs = k_pool.shape[2]
    scale = D ** -0.5 if scale is None else scale
    out = np.zeros((n, H, D))
    for s in range(n):
        L = int(context_lens[s])
        rows = [(int(block_tables[s][j // bs]), j % bs) for j in range(L)]
        for h in range(H):
            k = np.array([k_pool[b, h, r] for b, r in rows], dtype=np.float64).reshape(L, D)
            v = np.array([v_pool[b, h, r] for b, r in rows], dtype=np.float64).reshape(L, D)
            out[s, h] = attention(q[s, h], k, v, scale)
    return out


# ------------------------------------------------------------------ routing harness


def route_topk(logits: np.ndarray, k: int):
    """train/model.py:158-162: softmax in fp32, top-k (largest first, lower index on
    ties), renormalised weights."""
    x = np.asarray(logits, dtype=np.float32)
    x = x - x.max(axis=-1, keepdims=True)
    p = np.exp(x)
    p = p / p.sum(axis=-1, keepdims=True)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(p, order, axis=-1)
    return (w / w.sum(axis=-1, keepdims=True)).astype(np.float32), order.astype(np.int64)


def sort_by_expert(experts_idx: np.ndarray, n_experts: int):
    """kernels/moe_routing.py:116-130: (token_of_slot, counts, pos)."""
    T, k = experts_idx.shape
    flat = experts_idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=n_experts)
    pos = np.empty_like(order)
    pos[order] = np.arange(T * k)
    return order // k, counts, pos.reshape(T, k)


# ------------------------------------------------------------------ tolerances (BASELINE)


def close_bf16(out: np.ndarray, ref: np.ndarray) -> tuple[bool, float]:
    """|out - ref| <= 1e-2 + 1e-2 |ref| (rtol = atol = 1e-2 for bf16 outputs)."""
    err = np.abs(_f32(out) - _f32(ref)) - (1e-2 + 1e-2 * np.abs(_f32(ref)))
    return bool((err <= 0).all()), float(err.max()) if err.size else 0.0


def close_fp32(out: np.ndarray, ref: np.ndarray) -> tuple[bool, float]:
    """2 fp16 ULP-equivalent relative error: |out - ref| <= 2^-9 max(|ref|, rms(ref))."""
    out, ref = _f32(out), _f32(ref)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) if ref.size else 0.0
    bound = 2.0 ** -9 * np.maximum(np.abs(ref), rms)
    ratio = np.abs(out - ref) / np.maximum(bound, 1e-30)
    return bool((np.abs(out - ref) <= bound).all()), float(ratio.max()) if ratio.size else 0.0
