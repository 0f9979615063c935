// Skinny weight-only GEMM (2 <= M <= 16, 16-bit activations) on the 16-bit MFMA: the kernel
// and its launch templates. gemv_mfma.hip instantiates the INT4 kernels and holds the entry
// points, gemv_mfma8.hip the INT8 kernels: the two are compiled with different code
// generation options (csrc/build.py).
//
//
// One v_mfma_f32_16x16x32 multiplies 16 weight rows n by all M (<= 16) activation
// rows at once, so the weights stream from HBM exactly once whatever M is. (The
// VALU GEMV keeps x in registers and re-reads the weights for every 4 rows of x.)
//
// Block = WAVES wavefronts on the same R x 16 weight rows; wavefront w takes a
// contiguous share of the K steps and the partial sums meet in LDS at the end.
// A step is one 16-byte weight load per lane per 16-row tile: 128 k for INT4
// (lane quarter q holds k [32q, 32q + 32) of the step), 64 k for INT8 ([16q, 16q+16)).
// Loads of up to U steps are issued before any arithmetic.
//
// Weights enter the MFMA without a subtract: an INT4 nibble v is OR-ed into the
// mantissa of bf16 128.0 / fp16 1024.0 (exact 128 + v / 1024 + v), an INT8 byte q as
// the exact integer q + 128. The offset is removed with the per-row sums of x, which
// one more MFMA against an all-ones operand produces in the same accumulator layout:
//   sum_k x (v - 8) = sum_k x (128 + v) - 136 sum_k x          (bf16; fp16: 1024, 1032).
// INT4 group scales multiply each step's partial sums (groups are multiples of 128; groups
// of 64 take steps of 64 k, a lane's 8 weight bytes per tile k [16q, 16q + 16));
// the INT8 row scale multiplies the reduced total.
//
// MFMA operands: weights are the "A" operand (rows n), x the "B" operand (columns m),
// so lane l accumulates D[n = 4 (l / 16) + i][m = l % 16], i = 0..3. Inside an INT4
// dword the nibbles are taken in k order 0,4,1,5,2,6,3,7 (one v_and_or per pair) and x
// is permuted to the same order with v_perm; INT8 and x stay in natural order.
#pragma once

#include <stdio.h>

#include <type_traits>

#include "wq.h"

namespace mls {

namespace {

template <typename AT> struct Mx;
template <> struct Mx<__bf16> {
  static constexpr uint32_t MAGIC = 0x43004300u;  // bf16 (128, 128)
  static constexpr float OFF4 = 136.0f;
  static constexpr uint32_t ONE2 = 0x3F803F80u;   // bf16 (1, 1)
  static constexpr float I8OFF = 128.0f;           // INT8 operands hold q + 128
  __device__ static __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // two exact small integers held in fp32 -> packed bf16 (truncation is exact here)
  __device__ static __forceinline__ uint32_t pack_int(float lo, float hi) {
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo),
                                 0x07060302u);
  }
};
template <> struct Mx<_Float16> {
  static constexpr uint32_t MAGIC = 0x64006400u;  // fp16 (1024, 1024)
  static constexpr float OFF4 = 1032.0f;
  static constexpr uint32_t ONE2 = 0x3C003C00u;   // fp16 (1, 1)
  static constexpr float I8OFF = 1152.0f;          // INT8 operands hold 1024 + q + 128
  __device__ static __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack_int(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  }
};

// buffer-load cache policy for the INT4 weights: non-temporal (read once; measured faster
// than the default: M = 4 4.60 against 5.05 us); the INT8 weights take the default (M = 16
// fp16 3.73 against 3.79 us)
constexpr int kNonTemporal = 2;

template <typename ST> __device__ __forceinline__ float ld_scale(const ST* s, int64_t i) {
  return (float)s[i];
}

// s_waitcnt vmcnt(N) (gfx9 encoding: low 4 bits, high 2 bits at 14; lgkm and exp counts
// left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt_le() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// 16-byte LDS-direct load: lane l writes LDS bytes [16 l, 16 l + 16) above `lds`
__device__ __forceinline__ void lds_load16x(__amdgpu_buffer_rsrc_t rs, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// INT4: the 8 nibbles of dword d (k = 0..7, even k low) -> MFMA operand in k order
// 0,4,1,5,2,6,3,7, each value the exact MAGIC + v. f and m hold 0x000F000F and MAGIC in
// registers made opaque once per kernel: with literal constants the compiler splits each
// (a & f) | m into v_and_b32 + v_or_b32 (gfx9 VOP3 encodings take no literal) instead of
// one v_and_or_b32.
__device__ __forceinline__ uint4 nib_operand(uint32_t d, uint32_t f, uint32_t m) {
  return make_uint4((d & f) | m, ((d >> 4) & f) | m, ((d >> 8) & f) | m, ((d >> 12) & f) | m);
}

// x chunk (8 16-bit values, k order 0..7) -> k order 0,4,1,5,2,6,3,7
__device__ __forceinline__ uint4 x_perm(const uint4& v) {
  return make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                    __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
}

// INT8: 8 bytes (two dwords, k order) -> 8 exact 16-bit values q + 128 (bf16), or
// 1024 + q + 128 for fp16: each biased byte u becomes the low byte of an fp16 whose high
// byte is 0x64, one v_perm per pair (Mx<AT>::I8OFF is what the operands add to q)
template <typename AT>
__device__ __forceinline__ uint4 byte_operand(uint32_t d0, uint32_t d1) {
  const uint32_t u = d0 ^ 0x80808080u, v = d1 ^ 0x80808080u;
  if constexpr (std::is_same_v<AT, _Float16>)
    return make_uint4(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u),
                      __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
  return make_uint4(Mx<AT>::pack_int((float)(u & 0xFFu), (float)((u >> 8) & 0xFFu)),
                    Mx<AT>::pack_int((float)((u >> 16) & 0xFFu), (float)(u >> 24)),
                    Mx<AT>::pack_int((float)(v & 0xFFu), (float)((v >> 8) & 0xFFu)),
                    Mx<AT>::pack_int((float)((v >> 16) & 0xFFu), (float)(v >> 24)));
}

// fp32 x piece (values 0..3 in a, 4..7 in b) -> its bf16 hi piece in a (the truncated upper
// halves) and lo piece in b (x - hi, rounded to nearest): x to about 2^-16 of its magnitude,
// the split pass's arithmetic for finite x
__device__ __forceinline__ void split_piece(uint4& a, uint4& b) {
  const uint32_t f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    h[t] = __builtin_amdgcn_perm(f[2 * t + 1], f[2 * t], 0x07060302u);
    bf16x2 v;
    v.x = (__bf16)(__uint_as_float(f[2 * t]) - __uint_as_float(f[2 * t] & 0xFFFF0000u));
    v.y = (__bf16)(__uint_as_float(f[2 * t + 1]) - __uint_as_float(f[2 * t + 1] & 0xFFFF0000u));
    l[t] = __builtin_bit_cast(uint32_t, v);
  }
  a = make_uint4(h[0], h[1], h[2], h[3]);
  b = make_uint4(l[0], l[1], l[2], l[3]);
}

// INT4 group scales of a wavefront's steps through LDS (SL): the wavefront's slice of the
// block's scale table, SLG groups from its first step's group g0 by 16 R rows, stored
// [group][row], one dword per scale (fp16 in the low half), so that a lane's 4
// consecutive rows are one 16-byte LDS read. It is filled by LDS-direct loads of one
// scale per lane (SLG * 16 R / 64 instructions),
// issued before any weight or activation load; the wavefront reads only its own slice,
// so its own vmcnt wait (which the compiler places before the first LDS read) is the
// only synchronisation. Without SL, every step loads each lane's 4 scales from global.
constexpr int SLG = 16;

// x through LDS (XL): with all of a wavefront's steps in one chunk, the wavefront first
// brings its K range of the M rows of x into its own LDS slice, [step][16 rows][KB k], by
// LDS-direct loads of whole 16-byte chunks (a row's step is 256 (INT4) or 128 (INT8)
// contiguous bytes, RPI rows per instruction), issued only for row groups below M. The
// MFMA operand reads then come from LDS: loaded straight into registers, every 16-byte
// x piece touched all of a row's cache lines at a quarter of their width, and the L1 and
// address units (not HBM) bounded the kernel. The 16-byte chunk index of row r is XOR-ed
// with r & (CH - 1) (conflict-free 16-row reads). Rows of the slice at or past M hold
// zeros or stale data; they feed only output columns m >= M, which are never stored.
//
// Split x (SPL, fp32 activations as bf16 hi + lo, mfma16.h): a holds the split rows of
// M <= 16 rows of x, the hi parts in rows 0..15 and the lo parts in rows 16..31; every MFMA
// on an x operand runs once on each part into the same accumulator, and the output is fp32.
// x comes straight from global (the LDS slice of both parts would not fit).
// XF (with SPL): a holds the M rows of x in fp32 (row stride lda floats) instead of split
// rows; each 8-value piece is loaded as two 16-byte halves and split in registers into its
// bf16 hi (truncated upper halves) and lo (x - hi, rounded to bf16) pieces, the split pass's
// arithmetic on finite x, so no separate split launch or workspace is needed.
template <int WBITS, typename AT, typename ST, int R, int WAVES, int U, bool SL, bool XL, bool S64, bool SPL = false,
          bool XF = false>
// One wavefront per SIMD is the design point (a grid of N / 16 blocks of WAVES
// wavefronts), so the compiler may spend registers on keeping a chunk's loads in flight.
// The files that instantiate this kernel are built with kernel-argument preloading (the
// first 14 dwords of the arguments arrive in SGPRs at wavefront start): everything the
// first loads need comes first, with the strides as 32-bit values (launch_one checks that
// they fit), and the output pointer and stride last.
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemv_mfma_kernel(
    const AT* __restrict__ a, const uint8_t* __restrict__ w, const ST* __restrict__ s, int K, int N, int M,
    int lda32, int ldw32, int ld_sn32, int ld_sg32, int group, std::conditional_t<SPL, float, AT>* __restrict__ c,
    int64_t ldc) {
  const int64_t lda = lda32, ldw = ldw32, ld_sn = ld_sn32, ld_sg = ld_sg32;
  using OT = std::conditional_t<SPL, float, AT>;
  static_assert(!(SPL && XL), "split x comes from global");
  static_assert(!XF || (SPL && std::is_same_v<AT, __bf16>), "fp32 x: split into bf16 parts");
  constexpr int XES = XF ? 4 : (int)sizeof(AT);  // bytes per x element in memory
  constexpr int XPARTS = SPL ? 2 : 1;
  constexpr bool W16 = WBITS == 8 || !S64;    // 16 weight bytes per lane and step (else 8)
  constexpr int KB = WBITS == 4 && W16 ? 128 : 64;  // k per step
  constexpr int NMF = WBITS == 4 && W16 ? 4 : 2;    // MFMAs per step and 16-row tile
  __shared__ f32x4 red[WAVES][R][64];
  // one dword per scale: an LDS-direct load of 2 bytes still advances 4 bytes per lane
  __shared__ __align__(16) uint32_t sls[SL ? WAVES : 1][SL ? SLG * 16 * R : 1];
  constexpr int XRB = KB * 2, CH = XRB / 16, RPI = 64 / CH;  // x bytes / 16-byte chunks per row-step
  static_assert(!XL || WAVES * U * 16 * XRB <= 128 * 1024, "x slices fit LDS");
  __shared__ __align__(16) uint8_t xls[XL ? WAVES : 1][XL ? U * 16 * XRB : 16];

  const int lane = threadIdx.x & 63;
  // wave-uniform by construction; readfirstlane lets the compiler keep the step
  // offsets in scalar registers (buffer-load soffset) instead of a waterfall loop
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int n_base = blockIdx.x * (16 * R);
  const int rows_w = min(16 * R, N - n_base);
  const int nsteps = K / KB;
  const int s_lo = (int)((int64_t)nsteps * wave / WAVES);
  const int s_hi = (int)((int64_t)nsteps * (wave + 1) / WAVES);

  // INT4 with SL: this wavefront's scale slice, before its other loads. Element e of the
  // slice is group g0 + e / (16 R) of block row e % (16 R); rows past N read zeros.
  const int spg = WBITS == 4 ? group / KB : 1;  // steps per group (INT4: a multiple of KB here)
  const float inv_spg = 1.0f / (float)spg;
  // group of step st: (st + 0.5) / spg is never within 0.5 / spg of an integer, far above
  // the fp32 rounding error at these sizes, so the truncation is exact
  auto group_of = [&](int st) __attribute__((always_inline)) { return (int)(((float)st + 0.5f) * inv_spg); };
  const int g0 = group_of(s_lo);
  if constexpr (WBITS == 4 && SL) {
    // the range is the block's true extent of s, ((rows_w - 1) ld_sn + (G - 1) ld_sg + 1)
    // scales, for any strides (transposed [G][N] scales, a broadcast row with ld_sn = 0)
    const int64_t s_ext = (int64_t)(rows_w - 1) * ld_sn + (int64_t)(K / group - 1) * ld_sg + 1;
    const __amdgpu_buffer_rsrc_t rss = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(s + (int64_t)n_base * ld_sn), (short)0, (int)(s_ext * (int64_t)sizeof(ST)), 0x00020000);
#pragma unroll
    for (int i = 0; i < SLG * 16 * R / 64; ++i) {
      const int e = 64 * i + lane, row = e % (16 * R), gl = e / (16 * R);
      const int off = (int)((row * ld_sn + (int64_t)(g0 + gl) * ld_sg) * (int64_t)sizeof(ST));
      auto* dst = (__attribute__((address_space(3))) void*)(&sls[wave][64 * i]);  // 4 bytes per lane
      if constexpr (sizeof(ST) == 2)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rss, dst, 2, off, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rss, dst, 4, off, 0, 0, 0);
    }
  }
  // rows of x past M and weight rows past N read as zeros (split x: the lo parts' M rows
  // start 16 rows down, through a descriptor of their own)
  const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a, (short)0, (int)(M * lda * (int64_t)XES), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsx_lo = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a + (SPL ? 16 * lda : 0)), (short)0, (int)(M * lda * (int64_t)sizeof(AT)), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (int64_t)n_base * ldw), (short)0, (int)(rows_w * ldw), 0x00020000);
  // this lane's byte offsets inside a step (x row m = r)
  const int x_off = r * (int)lda * XES + NMF * 16 * q * (XES / (int)sizeof(AT));
  int w_off[R];
#pragma unroll
  for (int t = 0; t < R; ++t) w_off[t] = (16 * t + r) * (int)ldw + (W16 ? 16 : 8) * q;
  // scale rows of this lane's accumulators: n = n_base + 16 t + 4 q + i
  int64_t s_row[R][4];
#pragma unroll
  for (int t = 0; t < R; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_row[t][i] = (int64_t)min(n_base + 16 * t + 4 * q + i, N - 1) * ld_sn;

  const uint4 ones = make_uint4(Mx<AT>::ONE2, Mx<AT>::ONE2, Mx<AT>::ONE2, Mx<AT>::ONE2);
  const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 acc[R];
#pragma unroll
  for (int t = 0; t < R; ++t) acc[t] = zero;
  f32x4 xsum = zero;  // INT8: sum_k x over this wave's steps
  uint32_t nib_f = 0x000F000Fu, nib_m = Mx<AT>::MAGIC;
  if constexpr (WBITS == 4) asm volatile("" : "+v"(nib_f), "+v"(nib_m));

  if constexpr (XL) {
    // the wavefront's x slice (one chunk: s_hi - s_lo <= U); steps past the range load
    // zeros (an offset past the buffer)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int soff = s_lo + u < s_hi ? (s_lo + u) * XRB : 0x7FFFFFF0;
#pragma unroll
      for (int rg = 0; rg < 16 / RPI; ++rg) {
        if (rg * RPI >= M) break;
        const int row = rg * RPI + lane / CH, lc = (lane % CH) ^ (row & (CH - 1));
        lds_load16x(rsx, &xls[wave][(u * 16 + rg * RPI) * XRB], row * (int)lda * (int)sizeof(AT) + lc * 16, soff);
      }
    }
  }
  for (int s0 = s_lo; s0 < s_hi; s0 += U) {
    uint4 wv[U][R], xv[U][NMF], xvl[SPL ? U : 1][SPL ? NMF : 1];
    float sc[WBITS == 4 ? U : 1][R][4];
    // All loads of the chunk first, and no branch between them and the MFMAs (a
    // conditional step lets the compiler sink its loads to the use and serialise the
    // chunk). A step past this wave's range re-reads its last step's weights and
    // reads x at an offset beyond the buffer, i.e. zeros, so it adds nothing.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = s0 + u < s_hi;  // wave-uniform
      const int st = live ? s0 + u : s_hi - 1;
      const int xs_off = live ? st * KB * XES : 0x7FFFFFF0;
#pragma unroll
      for (int t = 0; t < R; ++t)
        if constexpr (W16) {
          wv[u][t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsw, w_off[t], st * 64,
                                                                                     WBITS == 8 ? 0 : kNonTemporal));
        } else {
          const uint2 v2 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rsw, w_off[t], st * 32, kNonTemporal));
          wv[u][t] = make_uint4(v2.x, v2.y, 0u, 0u);
        }
      if constexpr (XF) {
        // piece j: fp32 values 0..3 into xv, 4..7 into xvl (split before use)
#pragma unroll
        for (int j = 0; j < NMF; ++j) {
          xv[u][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsx, x_off + 32 * j, xs_off, 0));
          xvl[u][j] =
              __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsx, x_off + 32 * j + 16, xs_off, 0));
        }
      } else if constexpr (!XL) {
#pragma unroll
        for (int j = 0; j < NMF; ++j)
          xv[u][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rsx, x_off + 16 * j, xs_off, 0));
        if constexpr (SPL) {
#pragma unroll
          for (int j = 0; j < NMF; ++j)
            xvl[u][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rsx_lo, x_off + 16 * j, xs_off, 0));
        }
      }
      if constexpr (WBITS == 4 && !SL) {
        const int64_t g = (int64_t)(st * KB / group) * ld_sg;
#pragma unroll
        for (int t = 0; t < R; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[u][t][i] = ld_scale(s, s_row[t][i] + g);
      }
    }
    // The LDS slices (scales, x) were filled by LDS-direct loads issued before the first
    // chunk's global loads. The compiler does not model the full extent of those loads,
    // so the wait is explicit: for everything but the chunk's own loads, issued after
    // them (vector loads complete in order; a count above 63 waits for more, which is
    // still correct).
    if constexpr (SL || XL) {
      constexpr int LPU = R + (XL ? 0 : XPARTS * NMF) + ((WBITS == 4 && !SL) ? 4 * R : 0);
      if (s0 == s_lo) wait_vmcnt_le<(U * LPU < 63 ? U * LPU : 63)>();
    }
    if constexpr (WBITS == 4 && SL) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int gl = min(group_of(min(s0 + u, s_hi - 1)) - g0, SLG - 1);
#pragma unroll
        for (int t = 0; t < R; ++t) {
          const uint4 v = *reinterpret_cast<const uint4*>(&sls[wave][gl * 16 * R + 16 * t + 4 * q]);
          const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (sizeof(ST) == 2)
              sc[u][t][i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d[i] & 0xFFFFu));
            else
              sc[u][t][i] = __builtin_bit_cast(float, d[i]);
          }
        }
      }
    }
    // lane (r, q)'s x pieces of step u from the LDS slice: chunks NMF q + j of row r (the k
    // of the register path)
    auto read_x = [&](int u) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < NMF; ++j)
        xv[u][j] = *reinterpret_cast<const uint4*>(
            &xls[wave][(u * 16 + r) * XRB + (((NMF * q + j) ^ (r & (CH - 1))) * 16)]);
    };
    if constexpr (XL) read_x(0);
    // INT4: step u's products (pp_st: weights against x; xs_st: ones against x, the row sums
    // behind the widening's offset), scaled into acc by scale_step one step later
    f32x4 xs_st[U], pp_st[U][R];
    auto scale_step = [&](int u) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < R; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[t][i] = fmaf(sc[u][t][i], fmaf(-Mx<AT>::OFF4, xs_st[u][i], pp_st[u][t][i]), acc[t][i]);
    };
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (XL) {
        // software pipeline: step u + 1's pieces are read before step u's arithmetic, which
        // hides their LDS latency; left to the compiler, every step's reads went ahead of all
        // arithmetic (A/B on one box: INT4 4096^2 M = 4 5.21 -> 5.08 us, M = 16 6.00 ->
        // 5.96; INT8 2048^2 M = 16 4.21 -> 4.05)
        if (u + 1 < U) read_x(u + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (XF) {
#pragma unroll
        for (int j = 0; j < NMF; ++j) split_piece(xv[u][j], xvl[u][j]);
      }
      if constexpr (WBITS == 4) {
        uint4 xo[XPARTS][NMF];
#pragma unroll
        for (int j = 0; j < NMF; ++j) {
          xo[0][j] = x_perm(xv[u][j]);
          if constexpr (SPL) xo[XPARTS - 1][j] = x_perm(xvl[u][j]);
        }
        f32x4 xs = zero;
#pragma unroll
        for (int h = 0; h < XPARTS; ++h)
#pragma unroll
          for (int j = 0; j < NMF; ++j) xs = Mx<AT>::mma(ones, xo[h][j], xs);
        xs_st[u] = xs;
#pragma unroll
        for (int t = 0; t < R; ++t) {
          const uint32_t d[4] = {wv[u][t].x, wv[u][t].y, wv[u][t].z, wv[u][t].w};
          f32x4 pp = zero;
#pragma unroll
          for (int j = 0; j < NMF; ++j) {
            const uint4 wop = nib_operand(d[j], nib_f, nib_m);
#pragma unroll
            for (int h = 0; h < XPARTS; ++h) pp = Mx<AT>::mma(wop, xo[h][j], pp);
          }
          pp_st[u][t] = pp;
        }
        // the previous step's group scaling, behind this step's MFMAs: its products have
        // long landed, where this step's own would hold the wavefront (one per SIMD) until
        // the MFMA chain drains
        if (u > 0) scale_step(u - 1);
      } else {
#pragma unroll
        for (int j = 0; j < NMF; ++j) {
          xsum = Mx<AT>::mma(ones, xv[u][j], xsum);
          if constexpr (SPL) xsum = Mx<AT>::mma(ones, xvl[u][j], xsum);
        }
#pragma unroll
        for (int t = 0; t < R; ++t) {
          const uint4 w0 = byte_operand<AT>(wv[u][t].x, wv[u][t].y), w1 = byte_operand<AT>(wv[u][t].z, wv[u][t].w);
          acc[t] = Mx<AT>::mma(w0, xv[u][0], acc[t]);
          acc[t] = Mx<AT>::mma(w1, xv[u][1], acc[t]);
          if constexpr (SPL) {
            acc[t] = Mx<AT>::mma(w0, xvl[u][0], acc[t]);
            acc[t] = Mx<AT>::mma(w1, xvl[u][1], acc[t]);
          }
        }
      }
    }
    if constexpr (WBITS == 4) scale_step(U - 1);
  }
  if constexpr (WBITS == 8) {
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(-Mx<AT>::I8OFF, xsum[i], acc[t][i]);
  }

  // ---- sum the wavefronts' partial results, scale (INT8), store
#pragma unroll
  for (int t = 0; t < R; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * 64; idx += 64 * WAVES) {
    const int t = idx / 64, l = idx % 64;
    f32x4 v = red[0][t][l];
#pragma unroll
    for (int ww = 1; ww < WAVES; ++ww) v += red[ww][t][l];
    const int m = l & 15, nb = n_base + 16 * t + 4 * (l >> 4);
    if (m >= M || nb >= N) continue;
    if constexpr (WBITS == 8) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] *= ld_scale(s, (int64_t)min(nb + i, N - 1) * ld_sn);
    }
    OT* dst = c + (int64_t)m * ldc + nb;
    if (nb + 3 < N && ((uintptr_t)dst & (sizeof(OT) * 4 - 1)) == 0) {
      store4<OT>(dst, v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nb + i < N) dst[i] = from_f32<OT>(v[i]);
    }
  }
}

// Tuning override for sweeps: MLS_GEMV_MFMA = "R,WAVES" (R in 1, 2; WAVES in 4, 8, 16; R = 2
// takes at most 8).
int env_pair(int& r, int& waves) {
  const char* v = getenv("MLS_GEMV_MFMA");
  if (!v || !*v) return 0;
  return sscanf(v, "%d,%d", &r, &waves) == 2;
}

template <int WBITS, typename AT, typename ST, int R, int WAVES, bool S64, bool SPL = false, bool XF = false>
int launch_one(const WqArgs& p) {
  constexpr int U = SPL ? 4 : 8;  // split x: both parts' registers for half the steps
  constexpr int KB = WBITS == 4 && !S64 ? 128 : 64;
  const int64_t blocks = cdiv(p.N, 16 * R);
  // the LDS scale slice: every wavefront's steps span at most SLG groups, and the slice's
  // global offsets stay in 32 bits
  static const bool sl_env = env_int("MLS_GEMV_MFMA_SL", 1) != 0;
  const int64_t nsteps = p.K / KB, per_wave = cdiv(nsteps, WAVES);
  const int64_t spg = WBITS == 4 ? p.group / KB : 1;
  const bool sl = WBITS == 4 && sl_env && cdiv(per_wave + spg - 1, spg) + 1 <= SLG &&
                  16 * R * p.ld_sn * (int64_t)sizeof(ST) < (1ll << 30) && (int64_t)(p.K / p.group) * p.ld_sg * (int64_t)sizeof(ST) < (1ll << 30);
  // x through LDS: one chunk per wavefront, and the wavefronts' slices within 128 KiB
  static const bool xl_env = env_int("MLS_GEMV_MFMA_XL", 1) != 0;
  constexpr bool XL_FITS = !SPL && WAVES * U * 16 * KB * 2 <= 128 * 1024;
  const bool xl = XL_FITS && xl_env && per_wave <= U;
  // the strides travel as 32-bit kernel arguments
  if (p.lda > 0x7FFFFFFF || p.ldw > 0x7FFFFFFF || p.ld_sn > 0x7FFFFFFF || p.ld_sg > 0x7FFFFFFF)
    return MLS_ERR_UNSUPPORTED;
  using OT = std::conditional_t<SPL, float, AT>;
  auto go = [&](auto slc, auto xlc) {
    hipLaunchKernelGGL((gemv_mfma_kernel<WBITS, AT, ST, R, WAVES, U, decltype(slc)::value, decltype(xlc)::value, S64,
                                         SPL, XF>),
                       dim3((unsigned)blocks), dim3(64 * WAVES), 0, p.stream, static_cast<const AT*>(p.a), p.w,
                       static_cast<const ST*>(p.s), (int)p.K, (int)p.N, (int)p.M, (int)p.lda, (int)p.ldw,
                       (int)p.ld_sn, (int)p.ld_sg, p.group, static_cast<OT*>(p.c), p.ldc);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  if constexpr (XL_FITS) {
    if (xl) {
      if (sl) go(T_{}, T_{});
      else go(F_{}, T_{});
      return MLS_OK;
    }
  }
  if (sl) go(T_{}, F_{});
  else go(F_{}, F_{});
  return MLS_OK;
}

template <int WBITS, typename AT, typename ST, bool S64, bool SPL = false, bool XF = false>
int launch_shape(const WqArgs& p) {
  constexpr int KB = WBITS == 4 && !S64 ? 128 : 64;
  const int64_t nsteps = p.K / KB;
  int r = 1, waves = nsteps >= 64 ? 8 : 4;  // about 8 steps (one chunk) per wavefront
  if (nsteps >= 128) waves = 16;
  // (twice the wavefronts with at most 4 steps each measured slower: M=16 6.05 -> 6.50 us)
  if constexpr (SPL) {  // split x: chunks of 4 steps, about one per wavefront
    waves = nsteps >= 64 ? 16 : nsteps >= 32 ? 8 : 4;
  }
  env_pair(r, waves);
  if constexpr (!SPL) {
    if (r == 2) {  // two tiles per wavefront: at most 8 wavefronts (16 spill)
      if (waves >= 8) return launch_one<WBITS, AT, ST, 2, 8, S64>(p);
      return launch_one<WBITS, AT, ST, 2, 4, S64>(p);
    }
  }
  if (waves == 16) return launch_one<WBITS, AT, ST, 1, 16, S64, SPL, XF>(p);
  if (waves == 8) return launch_one<WBITS, AT, ST, 1, 8, S64, SPL, XF>(p);
  return launch_one<WBITS, AT, ST, 1, 4, S64, SPL, XF>(p);
}

template <int WBITS, typename AT, bool S64 = false, bool SPL = false, bool XF = false>
int launch_st(const WqArgs& p) {
  return p.s_dt == MLS_F16 ? launch_shape<WBITS, AT, _Float16, S64, SPL, XF>(p)
                           : launch_shape<WBITS, AT, float, S64, SPL, XF>(p);
}

}  // namespace

// The INT8 kernels (gemv_mfma8.hip): p as checked by launch_gemv_mfma / launch_gemv_mfma_split.
int launch_gemv_mfma_int8(const WqArgs& p);
int launch_gemv_mfma_split_int8(const WqArgs& q);
int launch_gemv_mfma_f32_int8(const WqArgs& p);

}  // namespace mls
