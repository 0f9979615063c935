// Device code of the decode GEMV family (gemv.hip): the lane-level dequantising dot
// products shared by its kernels, and the body of the M = 1 / M = 2 kernel with 16-bit
// activations (gemv1_body), which gemv.hip wraps as gemv1_kernel. The body is a
// force-inlined device function so that a timing-only copy of the kernel (floor.hip,
// outside the library) can bracket exactly the same instructions with clock reads.
//
// Decode-shaped weight-only GEMM (small M): the HBM-bound family.
//
// Each wavefront owns R output columns n (weight rows) over the whole K. Lane l
// owns 16-byte weight chunks c = l + 64 j (j < CPL) of every one of its rows, so
// one load instruction covers 1 KiB of a row contiguously, and all R*CPL loads
// of a lane are issued before any arithmetic. The lane's slice of x (the same
// k range for every row) is loaded once and kept in registers, already laid out
// for the dot products, then reused across the R rows.
//
// Dequantization is folded into the dot products: a 16-byte INT4 chunk (32 k)
// lies inside one scale group, so  sum_k x_k (v_k - 8) s_g = s_g (sum_k x_k v'_k
// - off * sum_k x_k)  where v'_k = v_k + bias is produced by OR-ing the nibble into
// the mantissa of a 16-bit float constant (bf16 128.0 / fp16 1024.0): one
// v_and_or per two weights and one v_dot2 per two products. fp32 activations use
// exact byte->float converts and FMAs. INT8 converts the signed bytes exactly (bf16 and fp32
// x, no offset), or, for fp16 x, places u = q ^ 0x80 = q + 128 in an fp16's low byte.
// Each lane's partial sums are reduced across the wavefront at the end.
#pragma once

#include <type_traits>

#include "wq.h"

namespace mls {

__device__ __forceinline__ float load_scale(const void* s, int s_dt, int64_t i) {
  return s_dt == MLS_F16 ? (float)((const _Float16*)s)[i] : ((const float*)s)[i];
}

__device__ __forceinline__ float ub0(uint32_t v) { return (float)(v & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t v) { return (float)(v >> 24); }
// signed bytes of v (one v_cvt_f32_i32 with an SDWA sign-extended byte select each)
__device__ __forceinline__ float sb0(uint32_t v) { return (float)(signed char)v; }
__device__ __forceinline__ float sb1(uint32_t v) { return (float)(signed char)(v >> 8); }
__device__ __forceinline__ float sb2(uint32_t v) { return (float)(signed char)(v >> 16); }
__device__ __forceinline__ float sb3(uint32_t v) { return (float)((int32_t)v >> 24); }

template <typename AT> struct Half16;

template <> struct Half16<__bf16> {
  static constexpr uint32_t MAGIC4 = 0x43004300u;  // bf16 128.0 in both halves
  static constexpr float OFF4 = 136.0f;            // 128 + 8
  static constexpr uint32_t ONE2 = 0x3F803F80u;    // bf16 (1.0, 1.0)
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  // exact for the integers 0..255 this is used on
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  // INT8: the signed bytes H2, H2 + 1 of q as the exact pair (q, q'); code_offset is 0
  template <int H2>
  __device__ static __forceinline__ uint32_t byte_pair(uint32_t q) {
    if constexpr (H2 == 0) return pack2(sb0(q), sb1(q));
    else return pack2(sb2(q), sb3(q));
  }
};

template <> struct Half16<_Float16> {
  static constexpr uint32_t MAGIC4 = 0x64006400u;  // fp16 1024.0 in both halves
  static constexpr float OFF4 = 1032.0f;           // 1024 + 8
  static constexpr uint32_t ONE2 = 0x3C003C00u;    // fp16 (1.0, 1.0)
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  }
  // INT8: bytes H2, H2 + 1 of q as the exact pair (1024 + u, 1024 + u') of the biased codes
  // u = q + 128: each u becomes the low byte of an fp16 with high byte 0x64, one v_perm per
  // pair (code_offset is 1152 = 1024 + 128)
  template <int H2>
  __device__ static __forceinline__ uint32_t byte_pair(uint32_t q) {
    return __builtin_amdgcn_perm(0x64646464u, q ^ 0x80808080u, H2 == 0 ? 0x04010400u : 0x04030402u);
  }
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int WBITS, typename AT>
struct XSlot {
  static constexpr bool F32 = sizeof(AT) == 4;
  static constexpr int KC = WBITS == 4 ? 32 : 16;    // k per 16-byte weight chunk
  static constexpr int NV = F32 ? KC : KC / 2;       // registers per chunk of x
};

// The lane's x values for one weight chunk: XQ 16-byte pieces loaded raw, then laid
// out for the dot products (x_from_raw returns their sum). Loading and unpacking are
// separate so that every load of the kernel can be issued before the first wait.
template <int WBITS, typename AT>
struct XRaw {
  static constexpr int XQ = XSlot<WBITS, AT>::KC * (int)sizeof(AT) / 16;
  uint4 v[XQ];
};

template <int WBITS, typename AT>
__device__ __forceinline__ void load_x_raw(const AT* __restrict__ xrow, int c, XRaw<WBITS, AT>& raw) {
  constexpr int KC = XSlot<WBITS, AT>::KC;
  const uint4* src = reinterpret_cast<const uint4*>(xrow + (int64_t)c * KC);
#pragma unroll
  for (int q = 0; q < XRaw<WBITS, AT>::XQ; ++q) raw.v[q] = src[q];
}

template <int WBITS, typename AT>
__device__ __forceinline__ float x_from_raw(const XRaw<WBITS, AT>& raw, uint32_t* xr) {
  using S = XSlot<WBITS, AT>;
  constexpr int KC = S::KC;
  if constexpr (S::F32) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < KC / 4; ++q) {
      const uint4 v = raw.v[q];
      xr[4 * q + 0] = v.x;
      xr[4 * q + 1] = v.y;
      xr[4 * q + 2] = v.z;
      xr[4 * q + 3] = v.w;
      sum += (__uint_as_float(v.x) + __uint_as_float(v.y)) + (__uint_as_float(v.z) + __uint_as_float(v.w));
    }
    return sum;
  } else {
    using H = Half16<AT>;
    uint32_t d[KC / 2];
#pragma unroll
    for (int q = 0; q < KC / 8; ++q) {
      d[4 * q + 0] = raw.v[q].x;
      d[4 * q + 1] = raw.v[q].y;
      d[4 * q + 2] = raw.v[q].z;
      d[4 * q + 3] = raw.v[q].w;
    }
    if constexpr (WBITS == 4) {
      // sub-block b holds k 8b..8b+7 as pairs (x0,x1)(x2,x3)(x4,x5)(x6,x7); the
      // nibble unpack yields weights for (k0,k4)(k1,k5)(k2,k6)(k3,k7).
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        xr[4 * b + 0] = __builtin_amdgcn_perm(d[4 * b + 2], d[4 * b + 0], 0x05040100u);
        xr[4 * b + 1] = __builtin_amdgcn_perm(d[4 * b + 2], d[4 * b + 0], 0x07060302u);
        xr[4 * b + 2] = __builtin_amdgcn_perm(d[4 * b + 3], d[4 * b + 1], 0x05040100u);
        xr[4 * b + 3] = __builtin_amdgcn_perm(d[4 * b + 3], d[4 * b + 1], 0x07060302u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < KC / 2; ++q) xr[q] = d[q];
    }
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < S::NV; ++q) sum = H::dot2(xr[q], H::ONE2, sum);
    return sum;
  }
}

template <int WBITS, typename AT>
__device__ __forceinline__ float load_x_chunk(const AT* __restrict__ xrow, int c, uint32_t* xr) {
  XRaw<WBITS, AT> raw;
  load_x_raw<WBITS, AT>(xrow, c, raw);
  return x_from_raw<WBITS, AT>(raw, xr);
}

// (a & m) | c, which the compiler selects as one v_and_or_b32 when m and c are in
// registers. gfx9-family VOP3 encodings take no 32-bit literal, so with literal constants
// it splits this into v_and_b32 + v_or_b32; the callers pass m and c as values made
// opaque once per kernel. (Plain code rather than inline asm: the compiler must see the
// VALU write to insert the wait states an MFMA reading the result needs.)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) { return (a & m) | c; }

// sum_k x_k * u_k over one 16-byte weight chunk, where u_k is the code as widened
// (INT4: nibble + bias of the 16-bit path, or the raw nibble for fp32; INT8: q, or 1024 + q +
// 128 for fp16 x); code_offset<WBITS, AT>() times sum_k x_k is what u_k adds to the signed code.
// nib_mask / magic: 0x000F000F and the 16-bit path's bias pattern, held in registers.
template <int WBITS, typename AT>
__device__ __forceinline__ float chunk_dot(const uint4 wq, const uint32_t* xr, uint32_t nib_mask, uint32_t magic) {
  using S = XSlot<WBITS, AT>;
  const uint32_t q[4] = {wq.x, wq.y, wq.z, wq.w};
  float acc = 0.0f;
  if constexpr (WBITS == 4) {
    if constexpr (S::F32) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t lo = q[b] & 0x0F0F0F0Fu, hi = (q[b] >> 4) & 0x0F0F0F0Fu;
        const float* x = reinterpret_cast<const float*>(xr) + 8 * b;
        acc = fmaf(ub0(lo), x[0], acc);
        acc = fmaf(ub0(hi), x[1], acc);
        acc = fmaf(ub1(lo), x[2], acc);
        acc = fmaf(ub1(hi), x[3], acc);
        acc = fmaf(ub2(lo), x[4], acc);
        acc = fmaf(ub2(hi), x[5], acc);
        acc = fmaf(ub3(lo), x[6], acc);
        acc = fmaf(ub3(hi), x[7], acc);
      }
    } else {
      using H = Half16<AT>;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t p0 = and_or(q[b], nib_mask, magic);
        const uint32_t p1 = and_or(q[b] >> 4, nib_mask, magic);
        const uint32_t p2 = and_or(q[b] >> 8, nib_mask, magic);
        const uint32_t p3 = and_or(q[b] >> 12, nib_mask, magic);
        acc = H::dot2(p0, xr[4 * b + 0], acc);
        acc = H::dot2(p1, xr[4 * b + 1], acc);
        acc = H::dot2(p2, xr[4 * b + 2], acc);
        acc = H::dot2(p3, xr[4 * b + 3], acc);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if constexpr (S::F32) {
        const float* x = reinterpret_cast<const float*>(xr) + 4 * t;
        acc = fmaf(sb0(q[t]), x[0], acc);
        acc = fmaf(sb1(q[t]), x[1], acc);
        acc = fmaf(sb2(q[t]), x[2], acc);
        acc = fmaf(sb3(q[t]), x[3], acc);
      } else {
        using H = Half16<AT>;
        acc = H::dot2(H::template byte_pair<0>(q[t]), xr[2 * t + 0], acc);
        acc = H::dot2(H::template byte_pair<2>(q[t]), xr[2 * t + 1], acc);
      }
    }
  }
  return acc;
}

// The 16-bit operand pairs of one weight chunk, as chunk_dot forms them (INT4: 16 dwords
// of biased nibble pairs in k order (0,4)(1,5)(2,6)(3,7) per 8 k; INT8: 8 dwords of byte pairs),
// for reuse across several rows of x (16-bit activations only).
template <int WBITS, typename AT>
struct WPairs {
  static constexpr int NW = WBITS == 4 ? 16 : 8;
  uint32_t v[NW];
};

template <int WBITS, typename AT>
__device__ __forceinline__ void chunk_widen(const uint4 wq, uint32_t nib_mask, uint32_t magic, WPairs<WBITS, AT>& w) {
  using H = Half16<AT>;
  const uint32_t q[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    if constexpr (WBITS == 4) {
      w.v[4 * b + 0] = and_or(q[b], nib_mask, magic);
      w.v[4 * b + 1] = and_or(q[b] >> 4, nib_mask, magic);
      w.v[4 * b + 2] = and_or(q[b] >> 8, nib_mask, magic);
      w.v[4 * b + 3] = and_or(q[b] >> 12, nib_mask, magic);
    } else {
      w.v[2 * b + 0] = H::template byte_pair<0>(q[b]);
      w.v[2 * b + 1] = H::template byte_pair<2>(q[b]);
    }
  }
}

// the same sum as chunk_dot, from widened pairs
template <int WBITS, typename AT>
__device__ __forceinline__ float pairs_dot(const WPairs<WBITS, AT>& w, const uint32_t* xr) {
  using H = Half16<AT>;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < WPairs<WBITS, AT>::NW; ++i) acc = H::dot2(w.v[i], xr[i], acc);
  return acc;
}

template <int WBITS, typename AT>
constexpr float code_offset() {
  if constexpr (WBITS == 8) return std::is_same_v<AT, _Float16> ? 1152.0f : 0.0f;
  else if constexpr (sizeof(AT) == 4) return 8.0f;
  else return Half16<AT>::OFF4;
}

// code_offset times a chunk's x sum, what the widened codes add to the dot product; exactly
// 0 when they add nothing (the sum is then never used, and its dot products are not emitted)
template <int WBITS, typename AT>
__device__ __forceinline__ float offset_term(float xsum) {
  constexpr float OFF = code_offset<WBITS, AT>();
  if constexpr (OFF == 0.0f) return 0.0f;
  else return OFF * xsum;
}

template <typename ST>
__device__ __forceinline__ float scale_value(const ST* s, int64_t i) {
  return to_f32(s[i]);
}

// ------------------------------------------------------------------ M = 1, 16-bit activations
//
// The same lane layout and dot products as gemv_wq_kernel, with the loads shaped for the
// per-CU memory pipeline, which moves about 64 bytes per clock. Every wavefront of the
// kernel above reads all of x (as many bytes as its weights) and issues one 2-byte scale
// load per weight chunk, so a wavefront spent ~0.45 us only issuing its loads. Here:
//  - x goes to LDS once per block: each wavefront brings a quarter with LDS-direct loads
//    (buffer_load ... lds), issued before anything else;
//  - a wavefront's INT4 group scales (R rows x K/group, contiguous per row) go to its own
//    LDS slice with one or two LDS-direct dword loads;
//  - the weight rows are buffer loads whose row offset sits in an SGPR (no per-lane 64-bit
//    address arithmetic before the loads issue);
//  - one wait for the LDS-direct loads (they were issued first and complete first) and one
//    barrier, which falls inside the weights' HBM latency;
//  - the cross-lane sums of the R rows are reduced together (lane-half and 16-lane-row swaps,
//    then DPP moves within rows: wave_totals), and one lane per row writes that row's output.
// LDS: x in XI * 4 KiB (the LDS-direct loads past 2K bytes read zeros past the buffer), then
// 4 scale slices of R * s_dw dwords, each rounded up to SI whole 64-dword LDS-direct
// instructions.

template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_add_rows(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWMASK,
                                                                   0xF, false));
}

// Wave total into lanes 48..63 (row sums by DPP, then rows 0-2 into row 3 by row_bcast).
__device__ __forceinline__ float wave_total_dpp(float v) {
  v = lane_group_sum<16>(v);
  v = dpp_add_rows<0x142, 0xA>(v);  // row_bcast:15: rows 1, 3 += last lane of rows 0, 2
  v = dpp_add_rows<0x143, 0xC>(v);  // row_bcast:31: rows 2, 3 += lane 31 (rows 0 + 1)
  return v;
}

// Wave totals of V per-lane partials (V = 1, 2 or a multiple of 4), reduced together: a swap
// of lane halves and an add (swap_add<32>) leave each value's two halves summed in one half
// of a register (two values per register), a swap of 16-lane rows and an add the same per
// row (four values per register), and 4 DPP steps finish each row: 3 + 3 + 4 instructions
// for 4 values where a DPP reduction per value takes 4 x 10. Slot k of lane l holds value
// total_index<V>(l, k), -1 where the lane is not the one that writes it.
template <int V>
struct WaveTotals {
  static_assert(V == 1 || V == 2 || V % 4 == 0, "1, 2 or a multiple of 4 values");
  static constexpr int NT = V >= 4 ? V / 4 : 1;
  float t[NT];
};

template <int V>
__device__ __forceinline__ WaveTotals<V> wave_totals(const float (&p)[V]) {
  WaveTotals<V> out;
  if constexpr (V == 1) {
    out.t[0] = wave_total_dpp(p[0]);
  } else if constexpr (V == 2) {
    const float a = lane_group_sum<16>(swap_add<32>(p[0], p[1]));  // lanes 0-31: value 0, 32-63: 1
    out.t[0] = dpp_add_rows<0x142, 0xA>(a);                          // row_bcast:15: rows 1, 3 += rows 0, 2
  } else {
    float a[V / 2];
#pragma unroll
    for (int i = 0; i < V / 2; ++i) a[i] = swap_add<32>(p[2 * i], p[2 * i + 1]);  // value 2i | 2i + 1
#pragma unroll
    for (int j = 0; j < V / 4; ++j)
      out.t[j] = lane_group_sum<16>(swap_add<16>(a[2 * j], a[2 * j + 1]));  // rows: values 4j + {0, 2, 1, 3}
  }
  return out;
}

template <int V>
__device__ __forceinline__ int total_index(int lane, int k) {
  if constexpr (V == 1) return lane == 63 ? 0 : -1;
  else if constexpr (V == 2) return (lane & 31) == 31 ? lane >> 5 : -1;
  else {
    const int g = lane >> 4;
    return (lane & 15) == 15 ? 4 * k + (((g & 1) << 1) | (g >> 1)) : -1;
  }
}

// v[i] for a lane-dependent i < R (selects, no indexed register access)
template <int R>
__device__ __forceinline__ float pick(const float (&v)[R], int i) {
  float s = v[0];
#pragma unroll
  for (int r = 1; r < R; ++r) s = i == r ? v[r] : s;
  return s;
}

__device__ __forceinline__ void lds_direct16(__amdgpu_buffer_rsrc_t rs, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void lds_direct4(__amdgpu_buffer_rsrc_t rs, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 4, voff, soff, 0, 0);
}

// vmcnt(n) alone (expcnt and lgkmcnt left at their maxima), gfx9 encoding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

template <int WBITS, typename AT, typename ST, int CPL, int R, int XI, int SI, int MX>
__device__ __forceinline__ void gemv1_body(const AT* __restrict__ x, const uint8_t* __restrict__ w,
                                                  int ldw, int w_bytes, const ST* __restrict__ s, int s_row_bytes,
                                                  int s_bytes, int group, AT* __restrict__ y, int N, int K,
                                                  int s_dw, int lda_b, int M, int ldy) {
  // fp32 x (M = 1): staged in LDS as fp32, split in registers into bf16 hi (truncation) and
  // lo (x - hi, rounded) parts, each dotted as a row of bf16 x; the output is fp32
  constexpr bool XF32 = std::is_same_v<AT, float>;
  static_assert(!XF32 || MX == 1, "fp32 x: one row");
  using HT = std::conditional_t<XF32, __bf16, AT>;  // the dot products' 16-bit type
  using S = XSlot<WBITS, HT>;
  constexpr int KC = S::KC, NV = S::NV;
  constexpr int S_SLICE = 64 * SI;  // scale dwords per wavefront slice
  constexpr int XB = XI * 4096;     // LDS bytes per row of x
  __shared__ __attribute__((aligned(16))) uint8_t smem[MX * XB + (WBITS == 4 ? 4 * S_SLICE * 4 : 16)];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nchunks = K / KC;
  const int n0 = (blockIdx.x * 4 + wave) * R;

  // 1. x into LDS (a quarter per wavefront, 1 KiB per instruction) and this wavefront's
  //    scales into its slice: issued first, so they complete before any weight load. The
  //    instructions before the weight loads are kept to a minimum (one buffer descriptor
  //    per operand from the kernel arguments, row offsets in SGPRs, no per-lane clamps):
  //    each one delays the weight stream. XI instructions per wavefront cover XI * 4 KiB
  //    >= 2K bytes; those past x read zeros into LDS padding.
  const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (MX == 1 ? 0 : (M - 1) * lda_b) + K * (int)sizeof(AT), 0x00020000);
#pragma unroll
  for (int mi = 0; mi < MX; ++mi) {
    // rows past M repeat row M - 1 (computed, never stored); bytes past a row's K are
    // the next row's or zeros, and feed only chunks past K, whose terms are dropped
    const int xo = MX == 1 ? 0 : min(mi, M - 1) * lda_b;
#pragma unroll
    for (int i = 0; i < XI; ++i)
      lds_direct16(rsx, smem + mi * XB + wave * 1024 + i * 4096, lane * 16, xo + wave * 1024 + i * 4096);
  }
  uint8_t* sl = smem + MX * XB + wave * (S_SLICE * 4);
  ST srow_raw[R];
  if constexpr (WBITS == 4) {
    // slice = the R rows' s_dw scale dwords back to back (rows past N read zeros); lane q of
    // instruction i loads slice dword 64 i + q, row r = dword / s_dw found by compares (R <= 4);
    // the lanes past R * s_dw re-read the last dword into the slice's padding
    const __amdgpu_buffer_rsrc_t rss = __builtin_amdgcn_make_buffer_rsrc((void*)s, (short)0, s_bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < SI; ++i) {
      const int q = min(64 * i + lane, R * s_dw - 1);
      int r = 0;
#pragma unroll
      for (int t = 1; t < R; ++t) r += q >= t * s_dw;
      lds_direct4(rss, sl + 256 * i, r * s_row_bytes + (q - r * s_dw) * 4, n0 * s_row_bytes);
    }
  } else {
    // the row scales, loaded ahead of the weights (they return first) and made live below,
    // where the wait for the LDS-direct loads already covers them: left to the compiler,
    // each load sank into the storing lane's branch and cost a full memory round trip
    // after the reduction
#pragma unroll
    for (int r = 0; r < R; ++r) srow_raw[r] = s[min(n0 + r, N - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. every weight chunk of this lane: rows past N read zeros (past the descriptor's range);
  //    chunks past K read whatever follows in memory and their terms are dropped below. Cache
  //    policy: non-temporal, but the default for INT8 with one row of x (K = N = 4096, one box:
  //    INT4 3.36 us with the hint against 3.41 without; INT8 M = 1 4.66 against 4.58, M = 2
  //    5.28 against 5.32)
  constexpr int WCPOL = WBITS == 8 && MX == 1 ? 0 : 2;
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, w_bytes, 0x00020000);
  uint4 wv[R][CPL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      wv[r][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsw, lane * 16 + 1024 * j,
                                                                                 (n0 + r) * ldw, WCPOL));
  __builtin_amdgcn_sched_barrier(0);  // nothing below (e.g. the group division's setup) ahead of the loads

  // the slice index of each (row, chunk)'s group scale (a division by the runtime group
  // size), computed while the loads are in flight instead of after the barrier
  int sidx[R][CPL];
  if constexpr (WBITS == 4) {
    const int P = s_dw * 4 / (int)sizeof(ST);  // scales per slice row
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int g = ((lane + 64 * j) * KC) / group;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        sidx[r][j] = min(r * P + g, S_SLICE * 4 / (int)sizeof(ST) - 1);
        asm volatile("" : "+v"(sidx[r][j]));
      }
    }
  }

  // 3. the LDS-direct loads have landed once only the weight loads are outstanding; after
  //    the barrier every wavefront's quarter of x is there
  wait_vmcnt<R * CPL>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::"s"(y));  // the output pointer's kernel-argument load, here and not after the sums
  float srow[R];
  if constexpr (WBITS == 8) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      asm volatile("" : "+v"(srow_raw[r]));
      srow[r] = to_f32(srow_raw[r]);
    }
  }
  float sc[R][CPL];
  if constexpr (WBITS == 4) {
    const ST* st = reinterpret_cast<const ST*>(sl);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < CPL; ++j) sc[r][j] = to_f32(st[sidx[r][j]]);
  }
  if constexpr (XF32) {
    // lane's chunk j: KC fp32 values of x, 16-byte pieces q (8 values) as bf16 hi and lo
    XRaw<WBITS, HT> xh[CPL], xo[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint4* xl = reinterpret_cast<const uint4*>(smem + (lane + 64 * j) * KC * 4);
#pragma unroll
      for (int q = 0; q < XRaw<WBITS, HT>::XQ; ++q) {
        const uint4 a = xl[2 * q], b = xl[2 * q + 1];
        const uint32_t f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t hp[4], lp[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          hp[t] = __builtin_amdgcn_perm(f[2 * t + 1], f[2 * t], 0x07060302u);  // truncated halves
          const float l0 = __uint_as_float(f[2 * t]) - __uint_as_float(f[2 * t] & 0xFFFF0000u);
          const float l1 = __uint_as_float(f[2 * t + 1]) - __uint_as_float(f[2 * t + 1] & 0xFFFF0000u);
          lp[t] = Half16<HT>::pack2(l0, l1);
        }
        xh[j].v[q] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
        xo[j].v[q] = make_uint4(lp[0], lp[1], lp[2], lp[3]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t xrh[CPL][NV], xrl[CPL][NV];
    float osx[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      osx[j] = offset_term<WBITS, HT>(x_from_raw<WBITS, HT>(xh[j], xrh[j]) + x_from_raw<WBITS, HT>(xo[j], xrl[j]));
    uint32_t nib_mask = 0x000F000Fu, magic = 0;
    if constexpr (WBITS == 4) magic = Half16<HT>::MAGIC4;
    asm volatile("" : "+v"(nib_mask), "+v"(magic));
    float part[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        WPairs<WBITS, HT> wp;
        chunk_widen<WBITS, HT>(wv[r][j], nib_mask, magic, wp);
        const float d = (pairs_dot<WBITS, HT>(wp, xrh[j]) + pairs_dot<WBITS, HT>(wp, xrl[j])) - osx[j];
        const float t = WBITS == 4 ? fmaf(sc[r][j], d, acc) : acc + d;
        acc = (64 * (j + 1) > nchunks && lane + 64 * j >= nchunks) ? acc : t;
      }
      part[r] = acc;
    }
    const WaveTotals<R> tot = wave_totals<R>(part);
    const int rows = min(R, N - n0);
#pragma unroll
    for (int k = 0; k < WaveTotals<R>::NT; ++k) {
      const int r = total_index<R>(lane, k);
      if (r >= 0 && r < rows)
        reinterpret_cast<float*>(y)[n0 + r] = WBITS == 8 ? tot.t[k] * pick<R>(srow, r) : tot.t[k];
    }
  } else if constexpr (MX == 1) {
    // one row of x (the M = 1 GEMV)
    XRaw<WBITS, AT> xraw[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint4* xl = reinterpret_cast<const uint4*>(smem + (lane + 64 * j) * KC * (int)sizeof(AT));
#pragma unroll
      for (int q = 0; q < XRaw<WBITS, AT>::XQ; ++q) xraw[j].v[q] = xl[q];
    }
    __builtin_amdgcn_sched_barrier(0);

    // 4. dot products (as gemv_wq_kernel); a chunk past K adds nothing (its scale may be
    //    any bits, so the whole term is dropped, not multiplied by zero)
    uint32_t xr[CPL][NV];
    float osx[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) osx[j] = offset_term<WBITS, AT>(x_from_raw<WBITS, AT>(xraw[j], xr[j]));
    uint32_t nib_mask = 0x000F000Fu, magic = 0;
    if constexpr (WBITS == 4) magic = Half16<AT>::MAGIC4;
    asm volatile("" : "+v"(nib_mask), "+v"(magic));
    float part[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const float d = chunk_dot<WBITS, AT>(wv[r][j], xr[j], nib_mask, magic) - osx[j];
        const float t = WBITS == 4 ? fmaf(sc[r][j], d, acc) : acc + d;
        acc = (64 * (j + 1) > nchunks && lane + 64 * j >= nchunks) ? acc : t;
      }
      part[r] = acc;
    }

    // 5. wave totals of the R rows together; one lane per row writes it
    const WaveTotals<R> tot = wave_totals<R>(part);
    const int rows = min(R, N - n0);
#pragma unroll
    for (int k = 0; k < WaveTotals<R>::NT; ++k) {
      const int r = total_index<R>(lane, k);
      if (r >= 0 && r < rows) y[n0 + r] = from_f32<AT>(WBITS == 8 ? tot.t[k] * pick<R>(srow, r) : tot.t[k]);
    }
  } else {
    // MX rows of x: each weight chunk is widened once and dotted with every row
    XRaw<WBITS, AT> xraw[MX][CPL];
#pragma unroll
    for (int mi = 0; mi < MX; ++mi)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const uint4* xl = reinterpret_cast<const uint4*>(smem + mi * XB + (lane + 64 * j) * KC * (int)sizeof(AT));
#pragma unroll
        for (int q = 0; q < XRaw<WBITS, AT>::XQ; ++q) xraw[mi][j].v[q] = xl[q];
      }
    __builtin_amdgcn_sched_barrier(0);

    // 4. dot products (as gemv_wq_kernel); a chunk past K adds nothing (its scale may be
    //    any bits, so the whole term is dropped, not multiplied by zero)
    uint32_t xr[MX][CPL][NV];
    float osx[MX][CPL];
#pragma unroll
    for (int mi = 0; mi < MX; ++mi)
#pragma unroll
      for (int j = 0; j < CPL; ++j) osx[mi][j] = offset_term<WBITS, AT>(x_from_raw<WBITS, AT>(xraw[mi][j], xr[mi][j]));
    uint32_t nib_mask = 0x000F000Fu, magic = 0;
    if constexpr (WBITS == 4) magic = Half16<AT>::MAGIC4;
    asm volatile("" : "+v"(nib_mask), "+v"(magic));
    float part[MX][R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc[MX];
#pragma unroll
      for (int mi = 0; mi < MX; ++mi) acc[mi] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const bool past_k = 64 * (j + 1) > nchunks && lane + 64 * j >= nchunks;
        WPairs<WBITS, AT> wp;
        chunk_widen<WBITS, AT>(wv[r][j], nib_mask, magic, wp);
#pragma unroll
        for (int mi = 0; mi < MX; ++mi) {
          const float d = pairs_dot<WBITS, AT>(wp, xr[mi][j]) - osx[mi][j];
          const float t = WBITS == 4 ? fmaf(sc[r][j], d, acc[mi]) : acc[mi] + d;
          acc[mi] = past_k ? acc[mi] : t;
        }
      }
#pragma unroll
      for (int mi = 0; mi < MX; ++mi) part[mi][r] = acc[mi];
    }

    // 5. wave totals of the MX x R outputs together; one lane per output writes it
    float flat[MX * R];
#pragma unroll
    for (int mi = 0; mi < MX; ++mi)
#pragma unroll
      for (int r = 0; r < R; ++r) flat[mi * R + r] = part[mi][r];
    const WaveTotals<MX * R> tot = wave_totals<MX * R>(flat);
    const int rows = min(R, N - n0);
#pragma unroll
    for (int k = 0; k < WaveTotals<MX * R>::NT; ++k) {
      const int i = total_index<MX * R>(lane, k);
      const int mi = i / R, r = i % R;  // (a row of x past M: computed, never stored)
      if (i >= 0 && r < rows && mi < M)
        y[(int64_t)mi * ldy + n0 + r] = from_f32<AT>(WBITS == 8 ? tot.t[k] * pick<R>(srow, r) : tot.t[k]);
    }
  }
}

}  // namespace mls
