// Medium weight-only GEMMs (16 < M <= 256 whose tiled GEMM would not fill the GPU),
// 16-bit activations, on the 16-bit MFMA with every operand loaded straight into
// registers.
//
// Block = 4 wavefronts on one output tile of TM x TN 16 x 16 MFMA tiles (rows m of x by
// weight rows n). The K steps are split into 4 contiguous ranges, one per wavefront, so
// no operand byte is loaded twice inside a block and nothing is staged through LDS on
// the way in: per step a lane loads its 16-byte pieces of x and of the weights, which
// are already in MFMA operand layout. The 4 partial tiles meet in LDS once, at the end.
// D steps of loads are in flight at once (a ring of D register sets).
//
// Step = 64 k (INT8: a lane's 16 weight bytes are k [16q, 16q + 16) of its row) or
// 128 k (INT4: 16 bytes = k [32q, 32q + 32)), q = lane / 16. x pieces follow the same k:
// INT8 two 16-byte loads, INT4 four. Rows m >= M, rows n >= N and steps past a
// wavefront's range read zeros (buffer loads past the operand's range).
//
// Widening: INT8 bytes to exact 16-bit integers (6 VALU per 4 weights); INT4 nibbles are
// OR-ed into the mantissa of bf16 128.0 / fp16 1024.0 (one v_and_or per 2 weights, exact
// 128 + v / 1024 + v, dword j of a piece giving k order 0,4,1,5,2,6,3,7 with x permuted
// alike) and the offset is removed with x's sums over the step, which one more MFMA
// against an all-ones operand gives in the same accumulator layout:
//   sum_k x (v - 8) = sum_k x (128 + v) - 136 sum_k x    (fp16: 1024, 1032).
// INT4 group scales (group a multiple of 128, so a step lies in one group) multiply each
// step's partial sums in fp32 (groups of 64: steps of 64 k, a lane's 8 weight bytes
// k [16q, 16q + 16), so that a step again lies in one group); the block's scales come into LDS once, by LDS-direct loads
// issued right after the first two steps' operands. INT8 row scales multiply the reduced
// tile. The instructions before the first operand loads are kept to a minimum: each one
// delays the weight stream.
//
// The weight operand is MFMA "A" and x is "B", so lane l's accumulator holds
// C[n = 4 (l / 16) + i][m = l % 16], i = 0..3: 4 consecutive outputs of one row m.
#include <type_traits>

#include "mfma16.h"

namespace mls {

namespace {

// soffset of a step past a wavefront's range: every access falls outside the operands
constexpr int kPastEnd = 0x40000000;

template <typename AT> struct Nib;
template <> struct Nib<__bf16> {
  static constexpr uint32_t MAGIC = 0x43004300u;  // bf16 (128, 128)
  static constexpr float OFF = 136.0f;            // 128 + 8
  static constexpr uint32_t ONE2 = 0x3F803F80u;   // bf16 (1, 1)
};
template <> struct Nib<_Float16> {
  static constexpr uint32_t MAGIC = 0x64006400u;  // fp16 (1024, 1024)
  static constexpr float OFF = 1032.0f;
  static constexpr uint32_t ONE2 = 0x3C003C00u;   // fp16 (1, 1)
};

struct SmallArgs {
  const void* a;
  int lda, a_bytes;  // elements; bytes of the M rows
  const uint8_t* w;
  int ldw, w_bytes;  // bytes; bytes of the N rows
  const void* s;
  int ld_sn, ld_sg, group, s_bytes;  // scale strides (elements), INT4 group, bytes of s
  void* c;
  int ldc;
  int M, N, K;
  int m_tiles, G;  // row tiles; INT4 groups per weight row
  int m_out;       // split rows (fp32 x as bf16 hi + lo, mfma16.h): output rows, fp32 output
  // x slices in LDS (kernels with 8 or 16 wavefronts): byte offset of the first slice,
  // log2 of a slice row's 16-byte chunks (a slice row holds xs_steps steps of one x row)
  int x_lds, xs_log2, xs_steps;
};

__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
}
__device__ __forceinline__ uint4 ld16_nt(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 2));
}

// x piece (8 16-bit values, k order 0..7) -> k order 0,4,1,5,2,6,3,7
__device__ __forceinline__ uint4 perm_x(const uint4& v) {
  return make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                    __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
}

// (a & m) | c with m and c in registers: one v_and_or_b32
__device__ __forceinline__ uint32_t andor(uint32_t a, uint32_t m, uint32_t c) { return (a & m) | c; }

// x through LDS (XLS, the 8- and 16-wavefront kernels): loaded per lane in MFMA layout, a
// 16-byte x piece touched 16 rows' cache lines at a quarter of their width, and the address
// unit (TA busy ~14.8k cycles per CU at M = 128, N = K = 2048, most of it stalled on the
// L1, ~41 L1 accesses per load instruction) bounded the kernel. Each wavefront now brings
// its K range of the tile's 16 TM rows of x into its own LDS slice with LDS-direct
// loads of whole 16-byte chunks, row by row (consecutive lanes, consecutive chunks of a
// row), the chunk index XOR-ed with row & 7; the MFMA pieces are then read from LDS. Each
// wavefront reads only its own slice, so its own vmcnt wait is the only synchronisation.
template <int WBITS, typename AT, typename ST, int TM, int TN, int D, bool S64 = false, bool SPLIT = false, int WV = 4,
          bool XLS = false>
// The arguments the first loads need come first, as scalars: this file is built with
// kernel-argument preloading (the first 14 dwords arrive in SGPRs at wavefront start), so
// those loads issue without waiting for a scalar load of the arguments. p (not preloaded)
// holds the rest; its copies of these fields are not read.
__global__ __launch_bounds__(64 * WV) void gemm_small_kernel(const void* pa, const uint8_t* pw, int lda, int a_bytes,
                                                            int ldw, int w_bytes, int N, int K, int x_lds, int xs_log2,
                                                            const SmallArgs p) {
  using MM = Mfma16<AT>;
  // split rows: 16-row tiles 2t and 2t + 1 hold the hi and lo parts of output rows
  // m0 / 2 + 16 t .. + 15, added in the epilogue; the output is fp32
  using OT = std::conditional_t<SPLIT, float, AT>;
  static_assert(!SPLIT || TM % 2 == 0, "split rows pair 16-row tiles");
  constexpr bool I4 = WBITS == 4;
  static_assert(!S64 || I4, "64-k INT4 steps");
  constexpr int KS = I4 && !S64 ? 128 : 64;  // k per step
  constexpr int XP = I4 && !S64 ? 4 : 2;     // 16-byte x pieces per lane, step and row tile
  constexpr int WB = I4 && S64 ? 8 : 16;     // weight bytes per lane and step
  extern __shared__ __align__(16) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, q = lane >> 4;
  // grid: x = column tile (padded to a multiple of 8), y = row tile. Workgroups go to the 8
  // XCDs round-robin by linear id, so every row tile of a column tile lands on the same XCD
  // and the weight tile is fetched from HBM once.
  const int nt = blockIdx.x, mt = blockIdx.y;
  const int m0 = mt * 16 * TM, n0 = nt * 16 * TN;
  if (n0 >= N) return;  // padding column tile
  const int nsteps = K / KS;
  const int s_lo = nsteps * wave / WV, s_hi = nsteps * (wave + 1) / WV;

  // ---- operand descriptors and this lane's offsets (nothing else before the first loads)
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void*)pa, (short)0, a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc((void*)pw, (short)0, w_bytes, 0x00020000);
  int xo[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) xo[tm] = (m0 + 16 * tm + r16) * lda * 2 + XP * 16 * q;
  int wo[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) wo[tn] = (n0 + 16 * tn + r16) * ldw + WB * q;

  uint8_t* xsl = smem + x_lds + wave * ((16 * TM) << (xs_log2 + 4));

  struct Slot {
    uint4 x[XLS ? 1 : TM][XLS ? 1 : XP];
    uint4 w[TN];
  };
  auto load = [&](Slot& sl, int st) __attribute__((always_inline)) {
    const int live = st < s_hi;
    const int sx = live ? st * KS * 2 : kPastEnd, sw = live ? st * 4 * WB : kPastEnd;
    if constexpr (!XLS) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int h = 0; h < XP; ++h) sl.x[tm][h] = ld16(rsa, xo[tm] + 16 * h, sx);
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if constexpr (WB == 8) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rsw, wo[tn], sw, 2));
        sl.w[tn] = make_uint4(v.x, v.y, 0u, 0u);
      } else {
        // INT8 weights with the default cache policy (the reference's M = 128 shape: 6.19 ->
        // 5.94 us), INT4 non-temporal
        sl.w[tn] = I4 ? ld16_nt(rsw, wo[tn], sw) : ld16(rsw, wo[tn], sw);
      }
    }
  };
  Slot sl[D];
#pragma unroll
  for (int d = 0; d < D; ++d) load(sl[d], s_lo + d);
  __builtin_amdgcn_sched_barrier(0);

  // ---- XLS: this wavefront's x slice, [16 TM rows][2^xs_log2 chunks], right after the
  // ring's first weight loads: the weights come from HBM and the slice mostly from L2, so
  // issued first the weights' latency runs under the slice's transfer (issued after the
  // slice, they queued behind all of it: the reference's bench shape, INT8 M = 128, ~0.2 us)
  if constexpr (XLS) {
    const int cpr_mask = (1 << xs_log2) - 1;
    const int total = (16 * TM) << xs_log2;  // chunks of the slice
    for (int c0 = 0; c0 < total; c0 += 64) {
      const int sidx = c0 + lane, row = sidx >> xs_log2, cp = sidx & cpr_mask;
      const int cl = cp ^ (row & 7);  // logical chunk stored at physical slot cp
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (__attribute__((address_space(3))) void*)(xsl + c0 * 16), 16,
                                               (m0 + row) * lda * 2 + cl * 16, s_lo * KS * 2, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (XLS && !I4) {
    // every load so far (the compiler does not model the LDS-direct writes)
    __builtin_amdgcn_s_waitcnt(0 | 0x70 | 0xF00);
    asm volatile("" ::: "memory");
  }

  // the remaining arguments into SGPRs at once (one round of scalar loads, issued at entry
  // and waited for here, after the first loads)
  asm volatile("" ::"s"(p.s), "s"(p.ld_sn), "s"(p.group), "s"(p.s_bytes), "s"(p.c), "s"(p.ldc), "s"(p.M), "s"(p.G));

  // ---- INT4 group scales of the block's 16 TN rows into LDS ([row][group] in ST), issued
  // after the first two steps' operands: the first step waits for nearly all of those
  // anyway, and the LDS-direct loads complete after them. Row r of table dword d is
  // d / dw_row, computed in fp32 ((2d + 1) / (2 dw_row) is never within 2^-10 of an
  // integer, far above the rounding error for these sizes).
  constexpr int BN = 16 * TN;
  if constexpr (I4) {
    const __amdgpu_buffer_rsrc_t rss = __builtin_amdgcn_make_buffer_rsrc((void*)p.s, (short)0, p.s_bytes, 0x00020000);
    const int dw_row = p.G * (int)sizeof(ST) / 4;  // dwords per row (G * sizeof(ST) % 4 == 0)
    const float inv2 = 0.5f / (float)dw_row;
    for (int q0 = wave * 64; q0 < BN * dw_row; q0 += 64 * WV) {
      const int d = min(q0 + lane, BN * dw_row - 1);
      const int r = (int)((float)(2 * d + 1) * inv2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rss, (__attribute__((address_space(3))) void*)(smem + q0 * 4), 4,
                                               (n0 + r) * p.ld_sn * (int)sizeof(ST) + (d - r * dw_row) * 4, 0, 0,
                                               0);
    }
    __builtin_amdgcn_s_waitcnt(0 | 0x70 | 0xF00);  // vmcnt(0): the table and both steps' operands
    __builtin_amdgcn_s_barrier();
  }

  f32x4 acc[TN][TM];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint32_t nmask = 0x000F000Fu, magic = Nib<AT>::MAGIC;
  asm volatile("" : "+v"(nmask), "+v"(magic));
  constexpr bool F16I8 = !I4 && std::is_same_v<AT, _Float16> && !SPLIT;
  const uint32_t hi64 = 0x64646464u;  // the fp16 high byte of 1024 + u (F16I8)
  f32x4 xsum[TM];                     // F16I8: sum_k x of row tile tm over this wavefront's steps
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) xsum[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint4 ones = make_uint4(Nib<AT>::ONE2, Nib<AT>::ONE2, Nib<AT>::ONE2, Nib<AT>::ONE2);
  const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};

  // this lane's x pieces of step st: from the slot (registers) or the LDS slice
  auto x_piece = [&](const Slot& sl, int st, int tm, int h) __attribute__((always_inline)) -> uint4 {
    if constexpr (XLS) {
      // a step past the wavefront's range (the ring's last round) multiplies zeros, as the
      // register path's past-the-end loads do: its slice position holds another step's x
      const bool live = st < s_hi;  // wave-uniform
      const int row = 16 * tm + r16;
      const int cl = (live ? st - s_lo : 0) * (KS * 2 / 16) + XP * q + h;
      const uint4 v = *reinterpret_cast<const uint4*>(xsl + ((row << xs_log2) + (cl ^ (row & 7))) * 16);
      return live ? v : make_uint4(0u, 0u, 0u, 0u);
    } else {
      return sl.x[tm][h];
    }
  };

  auto compute = [&](const Slot& sl, int st) __attribute__((always_inline)) {
    if constexpr (I4) {
      constexpr int NJ = XP;  // weight dwords (8 nibbles each) per lane and step
      uint4 xpm[TM][NJ];
      f32x4 xs[TM];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) xpm[tm][j] = perm_x(x_piece(sl, st, tm, j));
        xs[tm] = zero;
#pragma unroll
        for (int j = 0; j < NJ; ++j) xs[tm] = MM::mma(ones, xpm[tm][j], xs[tm]);
      }
      // scales of rows n = n0 + 16 tn + 4 q + i for this step's group (clamped past K)
      const int g = min(st * KS / p.group, p.G - 1);
      const ST* sl_s = reinterpret_cast<const ST*>(smem);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t d[4] = {sl.w[tn].x, sl.w[tn].y, sl.w[tn].z, sl.w[tn].w};
        uint4 wop[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          wop[j] = make_uint4(andor(d[j], nmask, magic), andor(d[j] >> 4, nmask, magic),
                              andor(d[j] >> 8, nmask, magic), andor(d[j] >> 12, nmask, magic));
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = to_f32(sl_s[(16 * tn + 4 * q + i) * p.G + g]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
          f32x4 pp = zero;
#pragma unroll
          for (int j = 0; j < NJ; ++j) pp = MM::mma(wop[j], xpm[tm][j], pp);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[tn][tm][i] = fmaf(sc[i], fmaf(-Nib<AT>::OFF, xs[tm][i], pp[i]), acc[tn][tm][i]);
        }
      }
    } else if constexpr (F16I8) {
      // INT8 with fp16 x: u = q ^ 0x80 = q + 128 goes into the low byte of an fp16 whose
      // high byte is 0x64 (one v_perm per two weights): exactly 1024 + u = 1152 + q. The
      // 1152 sum_k x is removed after the loop, from x's row sums (an MFMA against ones).
      uint4 xv[TM][2];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        xv[tm][0] = x_piece(sl, st, tm, 0);
        xv[tm][1] = x_piece(sl, st, tm, 1);
        xsum[tm] = MM::mma(ones, xv[tm][0], xsum[tm]);
        xsum[tm] = MM::mma(ones, xv[tm][1], xsum[tm]);
      }
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t d[4] = {sl.w[tn].x ^ 0x80808080u, sl.w[tn].y ^ 0x80808080u, sl.w[tn].z ^ 0x80808080u,
                               sl.w[tn].w ^ 0x80808080u};
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[2 * j + 0] = __builtin_amdgcn_perm(hi64, d[j], 0x04010400u);
          o[2 * j + 1] = __builtin_amdgcn_perm(hi64, d[j], 0x04030402u);
        }
        const uint4 w0 = make_uint4(o[0], o[1], o[2], o[3]), w1 = make_uint4(o[4], o[5], o[6], o[7]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
          acc[tn][tm] = MM::mma(w0, xv[tm][0], acc[tn][tm]);
          acc[tn][tm] = MM::mma(w1, xv[tm][1], acc[tn][tm]);
        }
      }
    } else {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        uint32_t o[8];
        widen_int8<AT>(sl.w[tn], o);
        const uint4 w0 = make_uint4(o[0], o[1], o[2], o[3]), w1 = make_uint4(o[4], o[5], o[6], o[7]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
          acc[tn][tm] = MM::mma(w0, x_piece(sl, st, tm, 0), acc[tn][tm]);
          acc[tn][tm] = MM::mma(w1, x_piece(sl, st, tm, 1), acc[tn][tm]);
        }
      }
    }
  };

  for (int st = s_lo; st < s_hi; st += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      compute(sl[d], st + d);
      load(sl[d], st + d + D);
    }
  }

  if constexpr (F16I8) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) acc[tn][tm] -= 1152.0f * xsum[tm];
  }

  // ---- the WV partial tiles meet in LDS; each thread finishes TN * TM / WV accumulators
  __syncthreads();  // (INT4: every wavefront is done with the scale table the buffer reuses)
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [WV][TN][TM][64]
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) red[((wave * TN + tn) * TM + tm) * 64 + lane] = acc[tn][tm];
  __syncthreads();
  OT* c = static_cast<OT*>(p.c);
  constexpr int TMO = SPLIT ? TM / 2 : TM;  // output row tiles
  for (int slot = threadIdx.x; slot < TN * TMO * 64; slot += 64 * WV) {
    const int l = slot & 63, to = (slot >> 6) % TMO, tn = (slot >> 6) / TMO;
    f32x4 v;
    int m;
    if constexpr (SPLIT) {
      v = red[(tn * TM + 2 * to) * 64 + l] + red[(tn * TM + 2 * to + 1) * 64 + l];
#pragma unroll
      for (int ww = 1; ww < WV; ++ww)
        v += red[((ww * TN + tn) * TM + 2 * to) * 64 + l] + red[((ww * TN + tn) * TM + 2 * to + 1) * 64 + l];
      m = m0 / 2 + 16 * to + (l & 15);
    } else {
      v = red[(tn * TM + to) * 64 + l];
#pragma unroll
      for (int ww = 1; ww < WV; ++ww) v += red[((ww * TN + tn) * TM + to) * 64 + l];
      m = m0 + 16 * to + (l & 15);
    }
    const int nb = n0 + 16 * tn + 4 * (l >> 4);
    if (m >= (SPLIT ? p.m_out : p.M) || nb >= N) continue;
    if constexpr (!I4) {
      const ST* sv = static_cast<const ST*>(p.s);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] *= to_f32(sv[min(nb + i, N - 1)]);
    }
    OT* dst = c + (int64_t)m * p.ldc + nb;
    if (nb + 3 < N && ((uintptr_t)dst & (SPLIT ? 15 : 7)) == 0) {
      store4<OT>(dst, v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nb + i < N) dst[i] = from_f32<OT>(v[i]);
    }
  }
}

template <int WBITS, typename AT, typename ST, int TM, int TN, int D, bool S64, bool SPLIT, int WV>
int launch_small_wv(SmallArgs a, hipStream_t st) {
  constexpr bool XLS = WV >= 8;  // x slices in LDS (a wavefront count with few steps each)
  a.m_tiles = (int)cdiv(a.M, 16 * TM);
  const int64_t nt = cdiv(cdiv(a.N, 16 * TN), 8) * 8;
  const int red = WV * TN * TM * 64 * 16;
  int sc = WBITS == 4 ? 16 * TN * a.G * (int)sizeof(ST) + 64 * WV * 4 : 0;  // + padding of the last dword load
  if (a.m_tiles > 65535) return MLS_ERR_UNSUPPORTED;
  if constexpr (XLS) {
    // a slice row holds a power of two of steps (at least the most any wavefront has): a
    // power-of-two chunk count, so lanes find their row and chunk by shifts
    constexpr int KS = WBITS == 4 && !S64 ? 128 : 64;
    const int smax = (int)cdiv(a.K / KS, WV);
    int steps = 1;
    while (steps < smax) steps *= 2;
    const int chunks = steps * KS * 2 / 16;  // >= 8, a power of two
    a.xs_log2 = __builtin_ctz((unsigned)chunks);
    a.xs_steps = steps;
    a.x_lds = (sc + 255) / 256 * 256;
    sc = a.x_lds + WV * 16 * TM * chunks * 16;
    if (sc > 160 * 1024) return MLS_ERR_UNSUPPORTED;
  }
  auto kern = gemm_small_kernel<WBITS, AT, ST, TM, TN, D, S64, SPLIT, WV, XLS>;
  const int lds = red > sc ? red : sc;
  if (lds > 65536) {  // above the default dynamic LDS limit: raise it once per instantiation
    static bool attr_set = false;
    if (!attr_set) {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
        return MLS_ERR_UNSUPPORTED;
      attr_set = true;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)nt, (unsigned)a.m_tiles), dim3(64 * WV), lds, st, a.a, a.w, a.lda,
                     a.a_bytes, a.ldw, a.w_bytes, a.N, a.K, a.x_lds, a.xs_log2, a);
  return MLS_OK;
}

// Registers per lane a (TM, TN) tile keeps live: accumulators and the ring of D steps of
// operands (16-byte pieces: TM XP of x and TN of weights per step), 4 VGPRs each.
template <int WBITS, int TM, int TN, int D, bool S64>
constexpr int small_regs() {
  constexpr int XP = WBITS == 4 && !S64 ? 4 : 2;
  return 4 * TM * TN + 4 * D * (TM * XP + TN);
}

// Wavefronts per block: the K steps are split over them, so more wavefronts keep more
// steps in flight per CU. 16 wavefronts (four per SIMD, 128 VGPRs a lane) hold one step
// each in flight (D = 1: the other wavefronts of the SIMD cover the latency), 8 (256
// VGPRs) two, 4 two. MLS_SMALL_WAVES = 4, 8 or 16 forces a count (sweeps); a count whose
// registers or reduction buffer would not fit falls back to fewer wavefronts.
template <int WBITS, typename AT, typename ST, int TM, int TN, int D, bool S64, bool SPLIT = false>
int launch_small(SmallArgs a, hipStream_t st) {
  static const int force = env_int("MLS_SMALL_WAVES", 0);
  const int KS = WBITS == 4 && !S64 ? 128 : 64;
  const int nsteps = a.K / KS;
  // 8 wavefronts with x slices in LDS from 16 steps on (the reference's bench shape, 2048 x
  // 2048 at M = 128: INT8 8.46 -> 8.10 us, INT4 g64 10.24 -> 8.52 us; 16 wavefronts measured
  // 8.40 / 9.38 us)
  int wv = nsteps >= 16 ? 8 : 4;
  if (force == 4 || force == 8 || force == 16) wv = force;
  // (the partial tiles of all wavefronts meet in LDS: WV TN TM KiB within 128 KiB)
  int rc = MLS_ERR_UNSUPPORTED;
  if constexpr (small_regs<WBITS, TM, TN, 1, S64>() <= 56 && 16 * TN * TM <= 128)
    if (wv >= 16) rc = launch_small_wv<WBITS, AT, ST, TM, TN, 1, S64, SPLIT, 16>(a, st);
  if constexpr (small_regs<WBITS, TM, TN, 2, S64>() <= 112 && 8 * TN * TM <= 128)
    if (rc == MLS_ERR_UNSUPPORTED && wv >= 8) rc = launch_small_wv<WBITS, AT, ST, TM, TN, 2, S64, SPLIT, 8>(a, st);
  // (the x slices too large for LDS: 4 wavefronts, x in registers)
  if (rc == MLS_ERR_UNSUPPORTED) rc = launch_small_wv<WBITS, AT, ST, TM, TN, D, S64, SPLIT, 4>(a, st);
  return rc;
}

// Time model for a tile of TM x TN: every block loads K * (16 TM * 2 + 16 TN * bytes per
// weight) bytes through its CU's memory pipeline; blocks beyond one per CU run in
// further rounds.
double small_cost(int64_t M, int64_t N, int64_t K, int wbits, int tm, int tn) {
  const int64_t blocks = cdiv(M, 16 * tm) * cdiv(N, 16 * tn);
  const double rows_x = (double)(M < 16 * tm ? M : 16 * tm);  // x loads of rows past M are skipped
  const double per_block = (double)K * (rows_x * 2.0 + 16.0 * tn * (wbits == 4 ? 0.5 : 1.0));
  return (double)cdiv(blocks, 256) * per_block;
}

// Whether the 8-wavefront kernel's x slices of a TM-row-tile block fit in LDS (as
// launch_small_wv sizes them), i.e. whether a tile height keeps x out of the registers.
bool small_xls_fits(const SmallArgs& a, int wbits, bool s64, int tm, int tn, int ssz) {
  const int ks = wbits == 4 && !s64 ? 128 : 64;
  const int nsteps = a.K / ks;
  if (nsteps < 16) return false;  // 4 wavefronts, no slices
  int steps = 1;
  while (steps < (nsteps + 7) / 8) steps *= 2;
  const int sc = wbits == 4 ? 16 * tn * a.G * ssz + 64 * 8 * 4 : 0;
  return (sc + 255) / 256 * 256 + 8 * 16 * tm * (steps * ks * 2 / 16) * 16 <= 160 * 1024;
}

template <int WBITS, typename AT, typename ST, bool S64 = false, bool SPLIT = false>
int dispatch_small(SmallArgs a, hipStream_t st) {
  static const int force = env_int("MLS_SMALL_TILE", 0);  // TM * 10 + TN (sweeps)
  int best_tm = SPLIT ? 2 : 1, best_tn = 1;
  double best = 1e300;
  for (int tm = SPLIT ? 2 : 1; tm <= 4; tm *= 2)
    for (int tn = 1; tn <= 4; tn *= 2) {
      if (tm > (SPLIT ? 2 : 1) && a.M <= 16 * tm / 2) continue;  // a row tile mostly past M
      if (WBITS == 4 && tm * tn > 8) continue;      // INT4 4 x 4 would spill registers
      const double c = small_cost(a.M, a.N, a.K, WBITS, tm, tn);
      // the model counts bytes only; the widening of every weight, once per block, costs
      // VALU time on top. A taller tile within 30% of the best byte count is taken when its
      // x slices fit in LDS: each weight is then widened for twice the rows (the reference's
      // bench shape, 2048 x 2048 at M = 128: 1 x 4 -> 2 x 2 tiles, INT8 8.05 -> 6.80 us, INT4
      // g128 7.51 -> 6.91 us, g64 8.50 -> 7.33 us; across M = 32..256 x (2048^2, 4096^2,
      // 11008 x 4096) no shape measured slower than the bytes-only choice)
      const bool taller_tie = c <= best * 1.3 && tm > best_tm &&
                              small_xls_fits(a, WBITS, S64, tm, tn, (int)sizeof(ST));
      if (c < best * 0.999 || taller_tie) {
        best = c;
        best_tm = tm;
        best_tn = tn;
      }
    }
  if (force && (!SPLIT || force / 10 >= 2)) {
    best_tm = force / 10;
    best_tn = force % 10;
  }
  // ring depth 2: deeper rings (up to 8 steps in flight) measured slower at M = 4..128
#define MLS_SMALL(TM_, TN_) \
  if (best_tm == TM_ && best_tn == TN_) return launch_small<WBITS, AT, ST, TM_, TN_, 2, S64, SPLIT>(a, st)
  if constexpr (!SPLIT) {
    MLS_SMALL(1, 1); MLS_SMALL(1, 2); MLS_SMALL(1, 4);
  }
  MLS_SMALL(2, 1); MLS_SMALL(2, 2); MLS_SMALL(2, 4);
  MLS_SMALL(4, 1); MLS_SMALL(4, 2);
  if constexpr (WBITS == 8) MLS_SMALL(4, 4);
#undef MLS_SMALL
  return MLS_ERR_UNSUPPORTED;
}

}  // namespace

// m_out > 0: p.a holds split rows (bf16 hi + lo of fp32 activations, mfma16.h), p.M of
// them; the output is fp32 with m_out rows.
static int small_impl(int wbits, const WqArgs& p, int64_t m_out) {
  if (p.a_dt != MLS_BF16 && p.a_dt != MLS_F16) return MLS_ERR_UNSUPPORTED;
  if (m_out > 0 && (p.a_dt != MLS_BF16 || p.M % 32 != 0)) return MLS_ERR_UNSUPPORTED;
  // INT4 steps of 128 k (groups a multiple of 128) or of 64 k (groups of 64)
  const bool s64 = wbits == 4 && p.group % 128 != 0;
  const int KS = wbits == 4 && !s64 ? 128 : 64;
  if (p.K % KS != 0 || p.K < KS) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && p.group % 64 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || p.lda % 8 != 0 || !aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  // 32-bit buffer offsets below the past-the-end soffset
  if (p.M * p.lda * 2 >= kPastEnd / 2 || (p.N + 64) * p.ldw >= kPastEnd / 2) return MLS_ERR_UNSUPPORTED;
  SmallArgs a{};
  a.a = p.a; a.lda = (int)p.lda; a.a_bytes = (int)(p.M * p.lda * 2);
  a.w = p.w; a.ldw = (int)p.ldw; a.w_bytes = (int)(p.N * p.ldw);
  a.s = p.s; a.ld_sn = (int)p.ld_sn; a.ld_sg = (int)p.ld_sg; a.group = p.group;
  a.c = p.c; a.ldc = (int)p.ldc; a.M = (int)p.M; a.N = (int)p.N; a.K = (int)p.K;
  a.m_out = (int)m_out;
  const int ssz = p.s_dt == MLS_F16 ? 2 : 4;
  if (wbits == 4) {
    a.G = (int)(p.K / p.group);
    // scales through LDS as whole dwords per row: contiguous groups, dword-aligned rows,
    // and a table of 64 rows that fits beside the reduction buffer
    if (p.ld_sg != 1 || (a.G * ssz) % 4 != 0 || (p.ld_sn * ssz) % 4 != 0 || !aligned(p.s, 4))
      return MLS_ERR_UNSUPPORTED;
    if (64 * a.G * ssz + 1024 > 65536 || (p.N * p.ld_sn + a.G) * ssz >= kPastEnd / 2) return MLS_ERR_UNSUPPORTED;
    // the descriptor spans the scales that exist: row N - 1 starts at (N - 1) ld_sn and
    // holds G groups (ld_sn may be below G, e.g. 0 for one row broadcast to every n)
    a.s_bytes = (int)(((p.N - 1) * p.ld_sn + a.G) * ssz);
  }
  if (m_out > 0) {
    if (wbits == 4 && s64) return p.s_dt == MLS_F16 ? dispatch_small<4, __bf16, _Float16, true, true>(a, p.stream)
                                                    : dispatch_small<4, __bf16, float, true, true>(a, p.stream);
    if (wbits == 4) return p.s_dt == MLS_F16 ? dispatch_small<4, __bf16, _Float16, false, true>(a, p.stream)
                                             : dispatch_small<4, __bf16, float, false, true>(a, p.stream);
    return p.s_dt == MLS_F16 ? dispatch_small<8, __bf16, _Float16, false, true>(a, p.stream)
                             : dispatch_small<8, __bf16, float, false, true>(a, p.stream);
  }
  if (wbits == 4 && s64) {
    if (p.a_dt == MLS_BF16) return p.s_dt == MLS_F16 ? dispatch_small<4, __bf16, _Float16, true>(a, p.stream)
                                                     : dispatch_small<4, __bf16, float, true>(a, p.stream);
    return p.s_dt == MLS_F16 ? dispatch_small<4, _Float16, _Float16, true>(a, p.stream)
                             : dispatch_small<4, _Float16, float, true>(a, p.stream);
  }
  if (wbits == 4) {
    if (p.a_dt == MLS_BF16) return p.s_dt == MLS_F16 ? dispatch_small<4, __bf16, _Float16>(a, p.stream)
                                                     : dispatch_small<4, __bf16, float>(a, p.stream);
    return p.s_dt == MLS_F16 ? dispatch_small<4, _Float16, _Float16>(a, p.stream)
                             : dispatch_small<4, _Float16, float>(a, p.stream);
  }
  if (p.a_dt == MLS_BF16) return p.s_dt == MLS_F16 ? dispatch_small<8, __bf16, _Float16>(a, p.stream)
                                                   : dispatch_small<8, __bf16, float>(a, p.stream);
  return p.s_dt == MLS_F16 ? dispatch_small<8, _Float16, _Float16>(a, p.stream)
                           : dispatch_small<8, _Float16, float>(a, p.stream);
}

int launch_gemm_small(int wbits, const WqArgs& p) { return small_impl(wbits, p, 0); }

int launch_gemm_small_split(int wbits, const WqArgs& p, int64_t m_out) {
  return m_out > 0 ? small_impl(wbits, p, m_out) : MLS_ERR_UNSUPPORTED;
}

}  // namespace mls
