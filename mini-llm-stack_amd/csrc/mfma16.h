// Shared pieces of the 16-bit MFMA GEMM kernels: launch parameters, the MFMA
// wrappers, the exact widening of INT8 / INT4 / e4m3 chunks to 16-bit floats, the
// LDS swizzle, and the buffer load that writes LDS directly.
#pragma once

#include "wq.h"

namespace mls {

enum { A_RAW16 = 0, A_E4M3 = 1, A_E5M2 = 2 };
enum { B_INT8 = 0, B_INT4 = 1, B_E4M3 = 2 };

struct Mfma16Params {
  const void* a;
  int64_t lda;  // elements of A's storage type (16-bit, or bytes for e4m3)
  const uint8_t* b;
  int64_t ldb;  // bytes
  const void* s;  // INT8 [N] / INT4 [N][G] scales
  int s_dt;
  int64_t ld_sn, ld_sg;
  int group;
  float sa, sb;  // e4m3 per-tensor scales (used when the pointers are null)
  const float* sap;
  const float* sbp;
  int64_t sas, sbs;
  void* c;
  int64_t ldc;
  int M, N, K;
  int n_tiles, m_tiles;
  const int32_t* seg_off;  // grouped: expert row offsets [E + 1]
  int E;
  int64_t b_estride, s_estride;  // grouped: bytes / scale elements between experts
  const uint8_t* b2;              // grouped gate/up: the up matrix (b is the gate)
  const void* s2;
  int ksplit;                     // grouped: K split into this many partial products (0, 1: none)
  int64_t c_sstride;              // grouped split: elements between the partial outputs
  const int32_t* a_rows;          // grouped: sorted row m is row a_rows[m] of a (null: row m)
  int a_src_rows;                 // grouped: rows of a when a_rows is set
  int tile_gm;                    // dense: row tiles per run of the tile order (0: column-major)
  int m_out;                      // split rows (fp32 activations as bf16 hi + lo, split.hip): rows of
                                  // the output; a's M rows hold the hi and lo parts (0: not split)
};

// fp32 activations on the 16-bit matrix cores (split.hip): x = hi + lo, two bf16 rows per
// row of x, arranged so that row R of the split matrix is part (R >> 4) & 1 (0: hi, 1: lo)
// of row m = 16 (R >> 5) + (R & 15). A kernel whose 16-row MFMA tiles start at multiples of
// 32 then holds the hi and lo products of one output row in the same lane, in the
// accumulators of tiles 2j and 2j + 1, and adds them in its epilogue (fp32).
__host__ __device__ constexpr int split_row(int m, int part) { return 32 * (m >> 4) + 16 * part + (m & 15); }
inline int64_t split_rows(int64_t M) { return 32 * cdiv(M, 16); }

// x = hi + lo: hi = x truncated to bf16 (exact; never overflows), lo = x - hi (exact in
// fp32, below 2^-7 |x|), rounded to bf16 by the caller; non-finite x: hi = x (a NaN stays
// a quiet NaN), lo = 0.
__device__ __forceinline__ void split_f32(float x, float& hi, float& lo) {
  const uint32_t u = __float_as_uint(x);
  const bool nonfinite = (u & 0x7F800000u) == 0x7F800000u;
  // a NaN whose payload lies only in the low 16 bits stays a (quiet) NaN, not an infinity
  hi = __uint_as_float((u & 0xFFFF0000u) | (nonfinite && (u & 0x007FFFFFu) ? 0x00400000u : 0u));
  lo = nonfinite ? 0.0f : x - hi;
}


template <typename T> struct Mfma16;
template <> struct Mfma16<__bf16> {
  __device__ static __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <> struct Mfma16<_Float16> {
  __device__ static __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    f16x2 v;
    v.x = (_Float16)lo;
    v.y = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
};

__device__ __forceinline__ int swz(int row) { return row & 7; }

// Logical tile L (consecutive on one XCD after xcd_remap) -> (row tile, column tile). gm = 0:
// every row tile of a column tile in turn. gm > 0: runs of gm row tiles sweep all column
// tiles, so an XCD's 32 concurrent blocks share ~gm row tiles and ~32 / gm column tiles.
__device__ __forceinline__ void tile_order(int L, int m_tiles, int n_tiles, int gm, int& mt, int& nt) {
  if (gm <= 0) {
    nt = L / m_tiles;
    mt = L % m_tiles;
    return;
  }
  const int per = gm * n_tiles, first = (L / per) * gm, gsz = min(m_tiles - first, gm), r = L % per;
  mt = first + r % gsz;
  nt = r / gsz;
}

__device__ __forceinline__ float scale_at(const void* s, int s_dt, int64_t i) {
  return s_dt == MLS_F16 ? (float)((const _Float16*)s)[i] : ((const float*)s)[i];
}

__device__ __forceinline__ float u8f(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }

// Signed byte b of v as an exact fp32 (one SDWA convert with sign extension).
template <int B>
__device__ __forceinline__ float sbyte_f32(uint32_t v) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(v));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(v));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(v));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(v));
  return r;
}

// Two exact small integers (|v| <= 256) held as fp32 -> one dword of 16-bit floats.
// bf16: the fp32 of such an integer has zero low 16 bits, so its high half is exact.
template <typename MT>
__device__ __forceinline__ uint32_t pack_exact2(float lo, float hi) {
  if constexpr (sizeof(MT) == 2 && __is_same(MT, _Float16))
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  else
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x07060302u);
}

// 16 INT8 weights -> 16 exact 16-bit floats (8 dwords, k order): 6 VALU per 4 weights.
template <typename MT>
__device__ __forceinline__ void widen_int8(const uint4& q, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    o[2 * t + 0] = pack_exact2<MT>(sbyte_f32<0>(d[t]), sbyte_f32<1>(d[t]));
    o[2 * t + 1] = pack_exact2<MT>(sbyte_f32<2>(d[t]), sbyte_f32<3>(d[t]));
  }
}

// 32 INT4 weights (even k in the low nibble) -> 32 exact values v - 8 (16 dwords).
template <typename MT>
__device__ __forceinline__ void widen_int4(const uint4& q, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = d[t] & 0x0F0F0F0Fu;         // k = 8t + 0, 2, 4, 6
    const uint32_t hi = (d[t] >> 4) & 0x0F0F0F0Fu;  // k = 8t + 1, 3, 5, 7
#pragma unroll
    for (int b = 0; b < 4; ++b)
      o[4 * t + b] = Mfma16<MT>::pack2(u8f(lo, b) - 8.0f, u8f(hi, b) - 8.0f);
  }
}

// 16 e4m3 bytes -> 16 bf16 (8 dwords, k order); exact: e4m3 is a subset of bf16.
__device__ __forceinline__ void widen_e4m3(const uint4& q, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    o[2 * t + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[t], 1.0f, false));
    o[2 * t + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[t], 1.0f, true));
  }
}

// 16 e5m2 bytes -> 16 bf16; exact: e5m2 (5 exponent bits, 2 mantissa bits, subnormals
// down to 2^-16, infinities) is a subset of bf16.
__device__ __forceinline__ void widen_e5m2(const uint4& q, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    o[2 * t + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(d[t], 1.0f, false));
    o[2 * t + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(d[t], 1.0f, true));
  }
}


// One 16-byte global chunk per lane straight into LDS (buffer_load_dwordx4 ... lds): lane l
// writes LDS bytes [16 l, 16 l + 16) above `lds`.
// Rows [lo, hi) of segment e of a grouped launch, clamped to [0, M). The offsets live on
// the device and cannot be checked by the host without a sync: offsets that break the
// contract (negative, decreasing, past M_total) shrink or overlap segments, but never
// move an access outside the operands.
__device__ __forceinline__ void seg_rows(const Mfma16Params& p, int e, int& lo, int& hi) {
  lo = min(max(p.seg_off[e], 0), p.M);
  hi = min(max(p.seg_off[e + 1], lo), p.M);
}

__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t rs, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff,
                                           soff, 0, 0);
}

// The exact e4m3 / e5m2 GEMM on 256-row tiles with both operands kept as bytes in LDS
// (gemm_bytes.hip); c_dt: output type.
int launch_bytes_fp8(const Mfma16Params& p, hipStream_t st, bool a_e5m2, int c_dt);

// Grouped INT4 GEMM with one block per (expert row chunk, 128 columns) (gemm_grouped.hip);
// gate_up: the gate/up pair of a SwiGLU expert MLP (p.b/p.s gate, p.b2/p.s2 up), output
// silu(gate) * up.
int launch_grouped_seg(const Mfma16Params& p, hipStream_t st, bool bf16, bool gate_up);
// The same GEMM as ksplit fp32 partial products over equal K ranges (p.c is fp32,
// partial s at p.c + s * p.c_sstride). MLS_ERR_UNSUPPORTED unless each range is a
// multiple of 64 and of the group and its scales fit the 32-group LDS table.
int launch_grouped_partial(const Mfma16Params& p, hipStream_t st, bool bf16);
// K splits that give the down projection of an expert MLP (few column tiles) two
// blocks per CU; 1 when no split is needed or possible.
int grouped_splits(int64_t M, int E, int64_t N, int64_t K, int group);

}  // namespace mls
