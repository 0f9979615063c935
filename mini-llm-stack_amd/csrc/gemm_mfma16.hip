// Tiled GEMMs on the 16-bit MFMA (v_mfma_f32_16x16x32_{bf16,f16}), one engine for
//   - weight-only INT8 / INT4 prefill: bf16/fp16 activations x dequantized weights,
//   - the per-expert (grouped) INT4 variant for MoE,
//   - the exact e4m3 GEMM: both e4m3 operands widened to bf16 (exact) on the way
//     into LDS.
// The 16-bit MFMAs add the exact products with fp32 precision, so every result
// here is what an fp32 GEMM of the dequantized / decoded operands gives, up to
// fp32 summation order. (gfx950's fp8 MFMAs instead truncate each product of a group of
// 8 toward zero at 2^-13 of the group's largest before adding them: gemm_fp8.hip.)
//
// Block tile BM (rows m of A) x BN (rows n of B) x 64 (k), WM x WN wavefronts (4, or
// 8 = two per SIMD so that one wavefront's memory waits overlap the other's MFMAs).
// Per k-stage every thread issues the loads of its share of the stage after next
// (16-byte buffer loads; rows past the tile's valid range read as zeros) into one of
// two register sets, runs the MFMAs of the current stage out of LDS, widens the
// chunks of the next stage (loaded one stage earlier) to 16-bit floats (INT8: exact integers; INT4: exact v - 8;
// e4m3: exact values via v_cvt_scalef32_pk_bf16_fp8) and stores them into the other
// LDS buffer; one barrier per stage. LDS rows are 64 k = 128 bytes; the 16-byte
// chunk index is XOR-ed with row & 7, which measured free of bank conflicts on
// gfx950 for both the staging writes and the MFMA operand reads of this kernel.
//
// The B tile is the MFMA "A" operand, so each lane's accumulator holds 4
// consecutive n of one m and the epilogue writes 4 outputs per store. Scales:
// INT8 per n in the epilogue; INT4 per (n, group) on fp32 partial sums at every
// group boundary; e4m3 per m and per n (or per tensor) in the epilogue.
#include "mfma16.h"

namespace mls {

template <int AKIND, int BKIND, typename MT, typename OT, int BM, int BN, int WM, int WN,
          bool GROUPED, bool DEEP>
__global__ __launch_bounds__(64 * WM * WN) void mfma16_gemm_kernel(const Mfma16Params p) {
  constexpr int BK = 64;
  constexpr int NT = 64 * WM * WN;             // threads per block
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 16, TN = WTN / 16;  // MFMA tiles per wave
  static_assert((WM * WN == 4 || WM * WN == 8) && TM >= 1 && TN >= 1, "bad wave layout");
  constexpr int A_ESZ = AKIND == A_RAW16 ? 2 : 1;
  constexpr int A_CPR = BK * A_ESZ / 16;                  // 16-byte chunks per row per stage
  constexpr int B_CPR = BKIND == B_INT4 ? 2 : 4;
  constexpr int A_CH = BM * A_CPR, B_CH = BN * B_CPR;
  constexpr int A_PT = (A_CH + NT - 1) / NT;
  static_assert(B_CH % NT == 0, "BN too small for the weight staging");
  static_assert(!(BKIND == B_INT4) || BN <= NT, "one thread per group scale");
  constexpr int B_PT = B_CH / NT;
  constexpr int A_RSTEP = NT / A_CPR, B_RSTEP = NT / B_CPR;
  constexpr bool GS = BKIND == B_INT4;  // group scales on fp32 partial sums

  extern __shared__ __align__(16) uint8_t smem[];
  uint4* As = reinterpret_cast<uint4*>(smem);  // [2][BM][8] 16-byte chunks
  uint4* Bs = As + 2 * BM * 8;                  // [2][BN][8]
  float* sS = reinterpret_cast<float*>(Bs + 2 * BN * 8);  // INT4: [2][2][BN]

  // ---- which tile: consecutive logical ids share a B tile and sit on one XCD
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int nt = L / p.m_tiles, mt = L % p.m_tiles;
  int row_hi = p.M, m0;
  const uint8_t* bmat = p.b;
  const void* smat = p.s;
  if constexpr (GROUPED) {
    int e = 0, cum = 0, row_lo = 0;
    for (; e < p.E; ++e) {
      int lo, hi;
      seg_rows(p, e, lo, hi);
      const int t = (hi - lo + BM - 1) / BM;
      if (mt < cum + t) {
        row_lo = lo;
        row_hi = hi;
        break;
      }
      cum += t;
    }
    if (e == p.E) return;  // surplus block
    m0 = row_lo + (mt - cum) * BM;
    bmat += (int64_t)e * p.b_estride;
    smat = (const uint8_t*)smat + (int64_t)e * p.s_estride * (p.s_dt == MLS_F16 ? 2 : 4);
  } else {
    m0 = mt * BM;
  }
  const int n0 = nt * BN;
  const int N = p.N;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;

  // ---- staging descriptors
  const int rows_a = min(BM, row_hi - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + (int64_t)m0 * p.lda * A_ESZ), (short)0,
      (int)(rows_a * p.lda * A_ESZ), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(bmat + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb), 0x00020000);
  const int a_row0 = tid / A_CPR, a_cc = tid % A_CPR;
  const int b_row0 = tid / B_CPR, b_cc = tid % B_CPR;
  int a_off[A_PT], b_off[B_PT];
#pragma unroll
  for (int i = 0; i < A_PT; ++i) a_off[i] = (a_row0 + A_RSTEP * i) * (int)p.lda * A_ESZ + a_cc * 16;
#pragma unroll
  for (int i = 0; i < B_PT; ++i) b_off[i] = (b_row0 + B_RSTEP * i) * (int)p.ldb + b_cc * 16;
  const bool a_on = A_CH >= NT || tid < A_CH;
  const int64_t s_row = (int64_t)min(n0 + tid, N - 1) * p.ld_sn;

  // DEEP: two register sets of prefetched chunks; the loads of stage s go to set s & 1
  // two stages before the stage is computed, so every load has two stages of MFMA work
  // to arrive in. Otherwise one set, loaded one stage ahead (for tiles whose
  // accumulators leave no room for a second set).
  uint4 ra0[A_PT], rb0[B_PT], ra1[A_PT], rb1[B_PT];
  float rs00 = 0.f, rs01 = 0.f, rs10 = 0.f, rs11 = 0.f;

  auto load = [&](uint4 (&ra)[A_PT], uint4 (&rb)[B_PT], float& rs0, float& rs1, int k0)
      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i)
      if (a_on)
        ra[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsa, a_off[i], k0 * A_ESZ, 0));
#pragma unroll
    for (int i = 0; i < B_PT; ++i)
      rb[i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rsb, b_off[i], BKIND == B_INT4 ? k0 / 2 : k0, 0));
    if constexpr (GS) {
      if (tid < BN) {
        const int kc = min(k0, p.K - BK);  // a stage past the end reuses the last scales
        rs0 = scale_at(smat, p.s_dt, s_row + (int64_t)(kc / p.group) * p.ld_sg);
        rs1 = scale_at(smat, p.s_dt, s_row + (int64_t)((kc + 32) / p.group) * p.ld_sg);
      }
    }
  };
  auto store = [&](const uint4 (&ra)[A_PT], const uint4 (&rb)[B_PT], float rs0, float rs1, int buf)
      __attribute__((always_inline)) {
    uint4* as = As + buf * BM * 8;
    uint4* bs = Bs + buf * BN * 8;
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      if (!a_on) continue;
      const int row = a_row0 + A_RSTEP * i;
      if constexpr (AKIND == A_RAW16) {
        as[row * 8 + (a_cc ^ swz(row))] = ra[i];
      } else {
        uint32_t o[8];
        if constexpr (AKIND == A_E5M2) widen_e5m2(ra[i], o);
        else widen_e4m3(ra[i], o);
        as[row * 8 + ((2 * a_cc + 0) ^ swz(row))] = make_uint4(o[0], o[1], o[2], o[3]);
        as[row * 8 + ((2 * a_cc + 1) ^ swz(row))] = make_uint4(o[4], o[5], o[6], o[7]);
      }
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      const int row = b_row0 + B_RSTEP * i;
      if constexpr (BKIND == B_INT4) {
        uint32_t o[16];
        widen_int4<MT>(rb[i], o);
#pragma unroll
        for (int h = 0; h < 4; ++h)
          bs[row * 8 + ((4 * b_cc + h) ^ swz(row))] =
              make_uint4(o[4 * h + 0], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
      } else {
        uint32_t o[8];
        if constexpr (BKIND == B_INT8) widen_int8<MT>(rb[i], o);
        else widen_e4m3(rb[i], o);
        bs[row * 8 + ((2 * b_cc + 0) ^ swz(row))] = make_uint4(o[0], o[1], o[2], o[3]);
        bs[row * 8 + ((2 * b_cc + 1) ^ swz(row))] = make_uint4(o[4], o[5], o[6], o[7]);
      }
    }
    if constexpr (GS) {
      if (tid < BN) {
        sS[(buf * 2 + 0) * BN + tid] = rs0;
        sS[(buf * 2 + 1) * BN + tid] = rs1;
      }
    }
  };

  f32x4 acc[TN][TM];
  f32x4 accg[GS ? TN : 1][GS ? TM : 1];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (GS) {
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int lr = lane & 15, lk = lane >> 4;
  // MFMAs of one stage out of LDS buffer `buf` (k0 = first k of the stage)
  auto compute = [&](int buf, int k0, int ks_lo = 0, int ks_hi = 2) __attribute__((always_inline)) {
    const uint4* as = As + buf * BM * 8;
    const uint4* bs = Bs + buf * BN * 8;
#pragma unroll
    for (int ks = ks_lo; ks < ks_hi; ++ks) {
      const int ch = ks * 4 + lk;
      uint4 bop[TN], aop[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int row = wn0 + i * 16 + lr;
        bop[i] = bs[row * 8 + (ch ^ swz(row))];
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int row = wm0 + j * 16 + lr;
        aop[j] = as[row * 8 + (ch ^ swz(row))];
      }
      if constexpr (GS) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TM; ++j) accg[i][j] = Mfma16<MT>::mma(bop[i], aop[j], accg[i][j]);
        if ((k0 + 32 * (ks + 1)) % p.group == 0) {  // group ends: acc += s[n] * partial
          const float* sc = sS + (buf * 2 + ks) * BN + wn0 + 4 * lk;
#pragma unroll
          for (int i = 0; i < TN; ++i) {
            const float4 s4 = *reinterpret_cast<const float4*>(sc + i * 16);
#pragma unroll
            for (int j = 0; j < TM; ++j) {
              acc[i][j][0] = fmaf(s4.x, accg[i][j][0], acc[i][j][0]);
              acc[i][j][1] = fmaf(s4.y, accg[i][j][1], acc[i][j][1]);
              acc[i][j][2] = fmaf(s4.z, accg[i][j][2], acc[i][j][2]);
              acc[i][j][3] = fmaf(s4.w, accg[i][j][3], acc[i][j][3]);
              accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TM; ++j) acc[i][j] = Mfma16<MT>::mma(bop[i], aop[j], acc[i][j]);
      }
    }
  };

  // Stage s is computed from LDS buffer s & 1, filled at the end of stage s - 1.
  const int nk = p.K / BK;
  if constexpr (DEEP) {
    // register set s & 1 holds stage s; the loads of stage s + 2 are issued at the start of s
    load(ra0, rb0, rs00, rs01, 0);
    if (nk > 1) load(ra1, rb1, rs10, rs11, BK);
    store(ra0, rb0, rs00, rs01, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
      if (kt + 2 < nk) load(ra0, rb0, rs00, rs01, (kt + 2) * BK);
      compute(0, kt * BK);
      if (kt + 1 < nk) store(ra1, rb1, rs10, rs11, 1);
      __syncthreads();
      if (kt + 1 >= nk) break;
      if (kt + 3 < nk) load(ra1, rb1, rs10, rs11, (kt + 3) * BK);
      compute(1, (kt + 1) * BK);
      if (kt + 2 < nk) store(ra0, rb0, rs00, rs01, 0);
      __syncthreads();
    }
  } else {
    // The next stage's chunks are widened and stored between the two k-halves of the
    // current stage, so that work overlaps the MFMAs still in flight instead of
    // running alone before the barrier. The loads and the store run unconditionally:
    // in the last stage they fetch k >= K (buffer loads return zeros past the
    // operand, group-scale indices are clamped) into the buffer nobody reads again.
    load(ra0, rb0, rs00, rs01, 0);
    store(ra0, rb0, rs00, rs01, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      load(ra0, rb0, rs00, rs01, (kt + 1) * BK);
      compute(buf, kt * BK, 0, 1);
      __builtin_amdgcn_sched_barrier(0);
      store(ra0, rb0, rs00, rs01, buf ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(buf, kt * BK, 1, 2);
      __syncthreads();
    }
  }

  // ---- epilogue: acc[i][j][r] = C[m = m0+wm0+16j+lr][n = n0+wn0+16i+4lk+r]
  OT* c = static_cast<OT*>(p.c);
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn0 + i * 16 + 4 * lk;
    float sn[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = min(nb + r, N - 1);
      if constexpr (BKIND == B_INT8) sn[r] = scale_at(smat, p.s_dt, n);
      if constexpr (BKIND == B_E4M3) sn[r] = p.sbp ? p.sbp[(int64_t)n * p.sbs] : p.sb;
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int m = m0 + wm0 + j * 16 + lr;
      if (m >= row_hi) continue;
      float sm = 1.f;
      if constexpr (BKIND == B_E4M3) sm = p.sap ? p.sap[(int64_t)m * p.sas] : p.sa;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = BKIND == B_E4M3 ? acc[i][j][r] * (sm * sn[r]) : acc[i][j][r] * sn[r];
      OT* dst = c + (int64_t)m * p.ldc + nb;
      if (nb + 3 < N && (p.ldc % 4) == 0) {
        store4<OT>(dst, v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) dst[r] = from_f32<OT>(v[r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Weight-only GEMM with the activation tile brought into LDS by buffer loads that
// write LDS directly (buffer_load_dwordx4 ... lds): 16-bit activations need no
// widening, so their stage costs no staging registers and no ds_write. Lane l of a
// wavefront fills LDS slot base + l and loads the global chunk that belongs there
// under the row & 7 swizzle. The weights are still staged through registers (widened
// to 16-bit on the way). Per stage s, in this order:
//   1. store stage s + 1's weights (loaded during stage s - 1) into the other buffer,
//   2. issue the loads of stage s + 2's weights,
//   3. read every operand of stage s from LDS,
//   4. issue the activation loads of stage s + 1 into the other buffer,
//   5. the MFMAs, then the barrier.
// The compiler keeps LDS reads behind pending LDS-direct loads; with this order the
// only such wait is the barrier's own, after the MFMAs have covered the load.

template <int BKIND, typename MT, typename OT, int BM, int BN, int WM, int WN, bool GROUPED, bool SPLIT = false>
__global__ __launch_bounds__(64 * WM * WN) void mfma16_adma_kernel(const Mfma16Params p) {
  constexpr int BK = 64;
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  static_assert(BKIND == B_INT8 || BKIND == B_INT4, "weight-only");
  constexpr int PW = BM * 8 / (64 * NW);  // activation loads per wavefront and stage
  static_assert(PW >= 1 && BM * 8 % (64 * NW) == 0, "activation slots");
  constexpr int B_CPR = BKIND == B_INT4 ? 2 : 4;
  constexpr int B_CH = BN * B_CPR;
  constexpr int B_PT = (B_CH + NT - 1) / NT;  // the last one guarded when B_CH % NT != 0
  constexpr int B_RSTEP = NT / B_CPR;
  constexpr bool GS = BKIND == B_INT4;
  static_assert(!GS || BN <= NT, "one thread per group scale");

  extern __shared__ __align__(16) uint8_t smem[];
  uint4* As = reinterpret_cast<uint4*>(smem);  // [2][BM][8]
  uint4* Bs = As + 2 * BM * 8;                  // [2][BN][8]
  float* sS = reinterpret_cast<float*>(Bs + 2 * BN * 8);  // INT4: [2][2][BN]

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int nt = L / p.m_tiles, mt = L % p.m_tiles;
  int row_hi = p.M, m0;
  const uint8_t* bmat = p.b;
  const void* smat = p.s;
  if constexpr (GROUPED) {
    int e = 0, cum = 0, row_lo = 0;
    for (; e < p.E; ++e) {
      int lo, hi;
      seg_rows(p, e, lo, hi);
      const int tcount = (hi - lo + BM - 1) / BM;
      if (mt < cum + tcount) {
        row_lo = lo;
        row_hi = hi;
        break;
      }
      cum += tcount;
    }
    if (e == p.E) return;  // surplus block
    m0 = row_lo + (mt - cum) * BM;
    bmat += (int64_t)e * p.b_estride;
    smat = (const uint8_t*)smat + (int64_t)e * p.s_estride * (p.s_dt == MLS_F16 ? 2 : 4);
  } else {
    m0 = mt * BM;
  }
  const int n0 = nt * BN;
  const int N = p.N;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;

  const int rows_a = min(BM, row_hi - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + (int64_t)m0 * p.lda * 2), (short)0, (int)(rows_a * p.lda * 2),
      0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(bmat + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb), 0x00020000);
  // activation slot s = (wave * PW + i) * 64 + lane: row s / 8, logical chunk (s % 8) ^ (row & 7)
  int a_off[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int s = (wave * PW + i) * 64 + lane, row = s >> 3, lc = (s & 7) ^ (row & 7);
    a_off[i] = row * (int)p.lda * 2 + lc * 16;
  }
  const int b_row0 = tid / B_CPR, b_cc = tid % B_CPR;
  int b_off[B_PT];
#pragma unroll
  for (int i = 0; i < B_PT; ++i) b_off[i] = (b_row0 + B_RSTEP * i) * (int)p.ldb + b_cc * 16;
  const int64_t s_row = (int64_t)min(n0 + tid, N - 1) * p.ld_sn;

  uint4 rb[B_PT];
  float rs0 = 0.f, rs1 = 0.f;
  auto dma_a = [&](int buf, int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PW; ++i) lds_load16(rsa, As + buf * BM * 8 + (wave * PW + i) * 64, a_off[i], k0 * 2);
  };
  auto load_b = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < B_PT; ++i)
      if (B_CH % NT == 0 || tid + NT * i < B_CH)
        rb[i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rsb, b_off[i], BKIND == B_INT4 ? k0 / 2 : k0, 0));
    if constexpr (GS) {
      if (tid < BN) {
        const int kc = min(k0, p.K - BK);  // a stage past the end reuses the last scales
        rs0 = scale_at(smat, p.s_dt, s_row + (int64_t)(kc / p.group) * p.ld_sg);
        rs1 = scale_at(smat, p.s_dt, s_row + (int64_t)((kc + 32) / p.group) * p.ld_sg);
      }
    }
  };
  auto store_b = [&](int buf) __attribute__((always_inline)) {
    uint4* bs = Bs + buf * BN * 8;
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      if (B_CH % NT != 0 && tid + NT * i >= B_CH) continue;
      const int row = b_row0 + B_RSTEP * i;
      if constexpr (BKIND == B_INT4) {
        uint32_t o[16];
        widen_int4<MT>(rb[i], o);
#pragma unroll
        for (int h = 0; h < 4; ++h)
          bs[row * 8 + ((4 * b_cc + h) ^ swz(row))] =
              make_uint4(o[4 * h + 0], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
      } else {
        uint32_t o[8];
        widen_int8<MT>(rb[i], o);
        bs[row * 8 + ((2 * b_cc + 0) ^ swz(row))] = make_uint4(o[0], o[1], o[2], o[3]);
        bs[row * 8 + ((2 * b_cc + 1) ^ swz(row))] = make_uint4(o[4], o[5], o[6], o[7]);
      }
    }
    if constexpr (GS) {
      if (tid < BN) {
        sS[(buf * 2 + 0) * BN + tid] = rs0;
        sS[(buf * 2 + 1) * BN + tid] = rs1;
      }
    }
  };

  f32x4 acc[TN][TM];
  f32x4 accg[GS ? TN : 1][GS ? TM : 1];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (GS) {
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int lr = lane & 15, lk = lane >> 4;
  const int nk = p.K / BK;
  // prologue: stage 0 in buffer 0, stage 1's weights in registers
  dma_a(0, 0);
  load_b(0);
  store_b(0);
  load_b(BK);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const int k0 = kt * BK;
    store_b(buf ^ 1);      // stage kt + 1 (past the end: harmless)
    load_b(k0 + 2 * BK);   // stage kt + 2
    uint4 aop[2][TM], bop[2][TN];
    const uint4* as = As + buf * BM * 8;
    const uint4* bs = Bs + buf * BN * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = ks * 4 + lk;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int row = wn0 + i * 16 + lr;
        bop[ks][i] = bs[row * 8 + (ch ^ swz(row))];
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int row = wm0 + j * 16 + lr;
        aop[ks][j] = as[row * 8 + (ch ^ swz(row))];
      }
    }
    float sc[GS ? 2 : 1][GS ? TN : 1][4];
    if constexpr (GS) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < TN; ++i) {
          const float4 s4 = *reinterpret_cast<const float4*>(sS + (buf * 2 + ks) * BN + wn0 + i * 16 + 4 * lk);
          sc[ks][i][0] = s4.x;
          sc[ks][i][1] = s4.y;
          sc[ks][i][2] = s4.z;
          sc[ks][i][3] = s4.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    dma_a(buf ^ 1, k0 + BK);  // stage kt + 1 (past the end: zeros / harmless)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if constexpr (GS) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TM; ++j) accg[i][j] = Mfma16<MT>::mma(bop[ks][i], aop[ks][j], accg[i][j]);
        if ((k0 + 32 * (ks + 1)) % p.group == 0) {  // group ends: acc += s[n] * partial
#pragma unroll
          for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(sc[ks][i][r], accg[i][j][r], acc[i][j][r]);
              accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
      } else {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TM; ++j) acc[i][j] = Mfma16<MT>::mma(bop[ks][i], aop[ks][j], acc[i][j]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the MFMAs stay ahead of the barrier's wait
    __syncthreads();
  }

  // ---- epilogue: acc[i][j][r] = C[m = m0+wm0+16j+lr][n = n0+wn0+16i+4lk+r]; split rows:
  // tiles 2j' and 2j' + 1 hold the hi and lo parts of output row (m0 + wm0) / 2 + 16j' + lr
  static_assert(!SPLIT || (!GROUPED && TM % 2 == 0 && (WTM % 32) == 0), "split rows pair whole 32-row groups");
  OT* c = static_cast<OT*>(p.c);
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn0 + i * 16 + 4 * lk;
    float sn[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (BKIND == B_INT8) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sn[r] = scale_at(smat, p.s_dt, min(nb + r, N - 1));
    }
#pragma unroll
    for (int j = 0; j < (SPLIT ? TM / 2 : TM); ++j) {
      const int m = SPLIT ? (m0 + wm0) / 2 + j * 16 + lr : m0 + wm0 + j * 16 + lr;
      if (m >= (SPLIT ? p.m_out : row_hi)) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = (SPLIT ? acc[i][2 * j][r] + acc[i][2 * j + 1][r] : acc[i][j][r]) * sn[r];
      OT* dst = c + (int64_t)m * p.ldc + nb;
      if (nb + 3 < N && (p.ldc % 4) == 0) {
        store4<OT>(dst, v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) dst[r] = from_f32<OT>(v[r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// INT8 weight-only GEMM (dense, 256-row tiles) with the weight widening overlapped with
// the MFMAs. The kernel above widens and stores the next stage's weights at the top of
// a stage, and both wavefronts of a SIMD reach that point together (the barrier aligns
// them), so their VALU work and their MFMAs never run at the same time; its barrier
// also drains the weight loads issued at the top of the same stage. Here, per stage s
// (activation and widened-weight tiles in separate double-buffered static LDS arrays,
// so the compiler can tell a pending LDS-direct load from the tiles it reads or writes):
//   1. read every operand of stage s from LDS,
//   2. issue the activation loads of stage s + 1 into the other A buffer,
//   3. the MFMAs of stage s, with stage s + 1's weights (in registers since stage
//      s - 1) widened and stored into the other B buffer in pieces between groups of
//      MFMAs,
//   4. issue stage s + 2's weight loads into the freed registers,
//   5. wait for this wavefront's loads but those weight loads, and barrier.
// The weights are staged in 8-byte pieces (8 k of one row), so that every thread
// issues the same number of loads (BN / 64 of them) whatever BN is: no thread-dependent
// branch in the loop, and one constant vmcnt.
// Measured at 2048 x 11008 x 4096 (same box, against the kernel above): MFMA busy 40% ->
// 45% of the cycles, VALU co-issued with MFMAs 0.2% -> 15% of the MFMA cycles, 220 ->
// 208 us.
typedef uint32_t lds16_t __attribute__((ext_vector_type(4)));

template <typename MT, typename OT, int BM, int BN, int WM, int WN, bool SPLIT = false>
__global__ __launch_bounds__(64 * WM * WN) void mfma16_w8_kernel(const Mfma16Params p) {
  constexpr int BK = 64;
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int PW = BM * 8 / NT;  // activation loads per wavefront and stage
  static_assert(PW >= 1 && BM * 8 % NT == 0, "activation slots");
  constexpr int B_PC = BN * 8;     // 8-byte weight pieces per stage
  static_assert(B_PC % NT == 0, "whole pieces per thread");
  constexpr int B_PT = B_PC / NT;  // per thread
  static_assert(B_PT <= 15, "vmcnt");
  constexpr int B_RSTEP = NT / 8;

  __shared__ __align__(16) uint4 As[2][BM * 8];
  __shared__ __align__(16) uint4 Bs[2][BN * 8];

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  int nt, mt;
  tile_order(L, p.m_tiles, p.n_tiles, p.tile_gm, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int M = p.M, N = p.N;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;

  const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + (int64_t)m0 * p.lda * 2), (short)0, (int)(rows_a * p.lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.b + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb), 0x00020000);
  int a_off[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int s = (wave * PW + i) * 64 + lane, row = s >> 3, lc = (s & 7) ^ (row & 7);
    a_off[i] = row * (int)p.lda * 2 + lc * 16;
  }
  // piece tid + NT i: row (tid >> 3) + B_RSTEP i, k 8 (tid & 7) .. + 7 of the stage; its
  // widened 16 bytes are LDS chunk (tid & 7) ^ (row & 7) of the row
  const int b_row0 = tid >> 3, b_kc = tid & 7;
  const int b_off0 = b_row0 * (int)p.ldb + b_kc * 8;
  const int b_lds0 = b_row0 * 8 + (b_kc ^ swz(b_row0));  // B_RSTEP is a multiple of 8

  uint2 rb[B_PT];
  auto load_b = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < B_PT; ++i)
      rb[i] = __builtin_bit_cast(
          uint2, __builtin_amdgcn_raw_buffer_load_b64(rsb, b_off0 + B_RSTEP * i * (int)p.ldb, k0, 0));
  };
  auto store_piece = [&](uint4* bs, int i) __attribute__((always_inline)) {
    const uint32_t d0 = rb[i].x, d1 = rb[i].y;
    bs[b_lds0 + B_RSTEP * 8 * i] =
        make_uint4(pack_exact2<MT>(sbyte_f32<0>(d0), sbyte_f32<1>(d0)), pack_exact2<MT>(sbyte_f32<2>(d0), sbyte_f32<3>(d0)),
                   pack_exact2<MT>(sbyte_f32<0>(d1), sbyte_f32<1>(d1)), pack_exact2<MT>(sbyte_f32<2>(d1), sbyte_f32<3>(d1)));
  };
  auto dma_a = [&](uint4* as, int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PW; ++i) lds_load16(rsa, as + (wave * PW + i) * 64, a_off[i], k0 * 2);
  };

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, lk = lane >> 4;
  const int nk = p.K / BK;

  // prologue: stage 0 in buffers 0, stage 1's weights in registers
  dma_a(As[0], 0);
  load_b(0);
#pragma unroll
  for (int i = 0; i < B_PT; ++i) store_piece(Bs[0], i);
  load_b(BK);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int r = kt & 1;
    // operand reads through an opaque base: otherwise the compiler may keep one address
    // register per tile read live across the loop
    uint32_t abase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)As[r];
    uint32_t bbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)Bs[r];
    asm volatile("" : "+v"(abase), "+v"(bbase));
    const auto* as = reinterpret_cast<const __attribute__((address_space(3))) lds16_t*>(abase);
    const auto* bs = reinterpret_cast<const __attribute__((address_space(3))) lds16_t*>(bbase);
    uint4* as_next = As[r ^ 1];
    uint4* bs_next = Bs[r ^ 1];
    const int k0 = kt * BK;
    uint4 aop[2][TM], bop[2][TN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = ks * 4 + lk;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int row = wn0 + i * 16 + lr;
        bop[ks][i] = __builtin_bit_cast(uint4, bs[row * 8 + (ch ^ swz(row))]);
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int row = wm0 + j * 16 + lr;
        aop[ks][j] = __builtin_bit_cast(uint4, as[row * 8 + (ch ^ swz(row))]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    dma_a(as_next, k0 + BK);  // stage kt + 1 (past the end: zeros / unused)
    __builtin_amdgcn_sched_barrier(0);
    {
      // the 2 TN TM MFMAs in B_PT groups; each group also widens and stores one weight
      // piece, which the scheduler interleaves with the group's MFMAs
      constexpr int PER = 2 * TN * TM / B_PT;
      static_assert(2 * TN * TM % B_PT == 0, "MFMA groups");
#pragma unroll
      for (int gi = 0; gi < B_PT; ++gi) {
#pragma unroll
        for (int x = gi * PER; x < (gi + 1) * PER; ++x) {
          const int ks = x / (TN * TM), i = (x / TM) % TN, j = x % TM;
          acc[i][j] = Mfma16<MT>::mma(bop[ks][i], aop[ks][j], acc[i][j]);
        }
        store_piece(bs_next, gi);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_b(k0 + 2 * BK);  // stage kt + 2 (past the end: harmless)
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    // everything but the weight loads just issued (vector loads complete in order),
    // and the widened-weight stores
    __builtin_amdgcn_s_waitcnt(B_PT | 0x70);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: acc[i][j][r] = C[m = m0+wm0+16j+lr][n = n0+wn0+16i+4lk+r]; split rows:
  // tiles 2j' and 2j' + 1 hold the hi and lo parts of output row (m0 + wm0) / 2 + 16j' + lr
  static_assert(!SPLIT || (TM % 2 == 0 && (WTM % 32) == 0), "split rows pair whole 32-row groups");
  OT* c = static_cast<OT*>(p.c);
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn0 + i * 16 + 4 * lk;
    float sn[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sn[r] = scale_at(p.s, p.s_dt, (int64_t)min(nb + r, N - 1) * p.ld_sn);
#pragma unroll
    for (int j = 0; j < (SPLIT ? TM / 2 : TM); ++j) {
      const int m = SPLIT ? (m0 + wm0) / 2 + j * 16 + lr : m0 + wm0 + j * 16 + lr;
      if (m >= (SPLIT ? p.m_out : M)) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = (SPLIT ? acc[i][2 * j][r] + acc[i][2 * j + 1][r] : acc[i][j][r]) * sn[r];
      OT* dst = c + (int64_t)m * p.ldc + nb;
      if (nb + 3 < N && (p.ldc % 4) == 0) {
        store4<OT>(dst, v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) dst[r] = from_f32<OT>(v[r]);
      }
    }
  }
}

template <typename MT, typename OT, int BN, bool SPLIT = false>
static int launch_w8(Mfma16Params p, hipStream_t st) {
  p.n_tiles = (int)cdiv(p.N, BN);
  static const int gm = env_int("MLS_TILE_GM", 4);  // row tiles per run of the tile order (0: column-major)
  p.tile_gm = gm;
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles;
  hipLaunchKernelGGL((mfma16_w8_kernel<MT, OT, 256, BN, 2, 4, SPLIT>), dim3((unsigned)blocks), dim3(512), 0, st, p);
  return check_launch("INT8 GEMM");
}

// ---------------------------------------------------------------------------
// INT4 weight-only GEMM (dense, 256-row tiles) on the INT8 kernel's schedule above: the
// activation tile arrives by LDS-direct loads, the next stage's weights are widened and
// stored between the current stage's MFMA groups, one barrier per stage. Per block and
// stage the weights are BN rows x 64 k = BN * 4 pieces of 8 bytes (16 k); a thread widens
// its piece's two dwords, one per k-step's MFMA group, each into one 16-byte LDS chunk
// (8 k) of exact 16 (v - 8) (x = d ^ 0x88888888 turns a nibble v into v ^ 8; masked into
// the high nibble of a byte it is the signed 16 (v - 8), one sign-extending convert per
// byte). Group scales by summation by parts: the block's table of coefficients
// c_g = (s_g - s_{g+1}) / 16 (c_{G-1} = s_{G-1} / 16; the 1/16 undoes the widening's
// factor) is computed once into LDS, the running products T are never cleared, and
// each group end adds c_g T to the result, one FMA per accumulator:
//   sum_g s_g P_g = sum_{g < G-1} (s_g - s_{g+1}) T_g + s_{G-1} T_{G-1},  T_g = P_0 + ... + P_g.
// Compared with the 128-row kernel (mfma16_adma_kernel), each widened weight feeds twice
// the rows, and a group end is one FMA per accumulator instead of an FMA and a clear.
constexpr int kW4MaxGroups = 64;  // coefficient table rows (32 KiB at BN = 128)

template <typename MT, typename OT, int BM, int BN, int WM, int WN, bool SPLIT = false>
__global__ __launch_bounds__(64 * WM * WN) void mfma16_w4_kernel(const Mfma16Params p) {
  constexpr int BK = 64;
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int PW = BM * 8 / NT;  // activation loads per wavefront and stage
  static_assert(PW >= 1 && BM * 8 % NT == 0, "activation slots");
  static_assert(BN * 4 == NT, "one 8-byte weight piece per thread and stage");
  constexpr int B_RSTEP = NT / 4;
  static_assert(B_RSTEP % 8 == 0, "swizzle");

  __shared__ __align__(16) uint4 As[2][BM * 8];
  __shared__ __align__(16) uint4 Bs[2][BN * 8];
  __shared__ __align__(16) float cT[kW4MaxGroups][BN];

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  int nt, mt;
  tile_order(L, p.m_tiles, p.n_tiles, p.tile_gm, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int M = p.M, N = p.N;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;

  const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + (int64_t)m0 * p.lda * 2), (short)0, (int)(rows_a * p.lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.b + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb), 0x00020000);
  int a_off[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int s = (wave * PW + i) * 64 + lane, row = s >> 3, lc = (s & 7) ^ (row & 7);
    a_off[i] = row * (int)p.lda * 2 + lc * 16;
  }
  // piece tid: row tid >> 2, k 16 (tid & 3) .. + 15 of the stage (8 bytes at k0 / 2 + 8 (tid & 3));
  // its dword h widens into LDS chunk 2 (tid & 3) + h of the row
  const int b_row = tid >> 2, b_kc = tid & 3;
  const int b_off = b_row * (int)p.ldb + b_kc * 8;
  const int b_lds0 = b_row * 8 + ((2 * b_kc) ^ swz(b_row));
  const int b_lds1 = b_row * 8 + ((2 * b_kc + 1) ^ swz(b_row));

  // the coefficient table: entry (g, n) for row n0 + n (rows past N repeat row N - 1, whose
  // outputs are not stored); consecutive threads read consecutive groups of one row
  const int G = p.K / p.group;
  for (int idx = tid; idx < G * BN; idx += NT) {
    const int n = idx / G, g = idx % G;
    const int64_t r = (int64_t)min(n0 + n, N - 1) * p.ld_sn;
    const float sg = scale_at(p.s, p.s_dt, r + (int64_t)g * p.ld_sg);
    const float sn = g + 1 < G ? scale_at(p.s, p.s_dt, r + (int64_t)(g + 1) * p.ld_sg) : 0.0f;
    cT[g][n] = (sg - sn) * 0.0625f;
  }

  uint2 rb;
  auto load_b = [&](int k0) __attribute__((always_inline)) {
    rb = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rsb, b_off, k0 / 2, 0));
  };
  // dword h of the piece -> one 16-byte chunk of 8 exact values 16 (v - 8), k order
  auto store_half = [&](uint4* bs, int h) __attribute__((always_inline)) {
    const uint32_t x = (h == 0 ? rb.x : rb.y) ^ 0x88888888u;
    const uint32_t hi = x & 0xF0F0F0F0u;         // byte b: k = 2b + 1
    const uint32_t lo = (x << 4) & 0xF0F0F0F0u;  // byte b: k = 2b
    bs[h == 0 ? b_lds0 : b_lds1] =
        make_uint4(pack_exact2<MT>(sbyte_f32<0>(lo), sbyte_f32<0>(hi)), pack_exact2<MT>(sbyte_f32<1>(lo), sbyte_f32<1>(hi)),
                   pack_exact2<MT>(sbyte_f32<2>(lo), sbyte_f32<2>(hi)), pack_exact2<MT>(sbyte_f32<3>(lo), sbyte_f32<3>(hi)));
  };
  auto dma_a = [&](uint4* as, int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PW; ++i) lds_load16(rsa, as + (wave * PW + i) * 64, a_off[i], k0 * 2);
  };

  f32x4 acc[TN][TM], tot[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      tot[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const int lr = lane & 15, lk = lane >> 4;
  const int nk = p.K / BK;

  // prologue: stage 0 in buffers 0, stage 1's weights in registers; the barrier also
  // publishes the coefficient table
  dma_a(As[0], 0);
  load_b(0);
  store_half(Bs[0], 0);
  store_half(Bs[0], 1);
  load_b(BK);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int r = kt & 1;
    uint32_t abase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)As[r];
    uint32_t bbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)Bs[r];
    asm volatile("" : "+v"(abase), "+v"(bbase));
    const auto* as = reinterpret_cast<const __attribute__((address_space(3))) lds16_t*>(abase);
    const auto* bs = reinterpret_cast<const __attribute__((address_space(3))) lds16_t*>(bbase);
    uint4* as_next = As[r ^ 1];
    uint4* bs_next = Bs[r ^ 1];
    const int k0 = kt * BK;
    uint4 aop[2][TM], bop[2][TN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = ks * 4 + lk;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int row = wn0 + i * 16 + lr;
        bop[ks][i] = __builtin_bit_cast(uint4, bs[row * 8 + (ch ^ swz(row))]);
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int row = wm0 + j * 16 + lr;
        aop[ks][j] = __builtin_bit_cast(uint4, as[row * 8 + (ch ^ swz(row))]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    dma_a(as_next, k0 + BK);  // stage kt + 1 (past the end: zeros / unused)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      // k-step ks's MFMAs with half of stage kt + 1's weights widened and stored beside them
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) tot[i][j] = Mfma16<MT>::mma(bop[ks][i], aop[ks][j], tot[i][j]);
      store_half(bs_next, ks);
      __builtin_amdgcn_sched_barrier(0);
      const int kend = k0 + 32 * (ks + 1);
      if (kend % p.group == 0) {  // group kend / group - 1 ends: acc += c_g T
        const int g = kend / p.group - 1;
#pragma unroll
        for (int i = 0; i < TN; ++i) {
          const float4 c4 = *reinterpret_cast<const float4*>(&cT[g][wn0 + i * 16 + 4 * lk]);
          const float c[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
          for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[i][j][q] = fmaf(c[q], tot[i][j][q], acc[i][j][q]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    load_b(k0 + 2 * BK);  // stage kt + 2 (past the end: harmless)
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    // everything but the weight load just issued (vector loads complete in order), and
    // the widened-weight stores
    __builtin_amdgcn_s_waitcnt(1 | 0x70);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: acc[i][j][q] = C[m = m0+wm0+16j+lr][n = n0+wn0+16i+4lk+q]; split rows:
  // tiles 2j' and 2j' + 1 hold the hi and lo parts of output row (m0 + wm0) / 2 + 16j' + lr
  static_assert(!SPLIT || (TM % 2 == 0 && (WTM % 32) == 0), "split rows pair whole 32-row groups");
  OT* c = static_cast<OT*>(p.c);
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn0 + i * 16 + 4 * lk;
    if (nb >= N) continue;
#pragma unroll
    for (int j = 0; j < (SPLIT ? TM / 2 : TM); ++j) {
      const int m = SPLIT ? (m0 + wm0) / 2 + j * 16 + lr : m0 + wm0 + j * 16 + lr;
      if (m >= (SPLIT ? p.m_out : M)) continue;
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = SPLIT ? acc[i][2 * j][q] + acc[i][2 * j + 1][q] : acc[i][j][q];
      OT* dst = c + (int64_t)m * p.ldc + nb;
      if (nb + 3 < N && (p.ldc % 4) == 0) {
        store4<OT>(dst, v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < N) dst[q] = from_f32<OT>(v[q]);
      }
    }
  }
}

// Whether mfma16_w4_kernel takes a dense INT4 GEMM: its coefficient table holds the groups
// (group a multiple of 32, G <= kW4MaxGroups); MLS_W4 = 0 keeps the 128-row kernel (A/B runs).
static bool w4_ok(const Mfma16Params& p) {
  static const bool on = env_int("MLS_W4", 1) != 0;
  return on && p.group % 32 == 0 && p.K % p.group == 0 && p.K / p.group <= kW4MaxGroups && p.M >= 256;
}

template <typename MT, typename OT, bool SPLIT = false>
static int launch_w4(Mfma16Params p, hipStream_t st) {
  constexpr int BN = 128;
  p.m_tiles = (int)cdiv(p.M, 256);
  p.n_tiles = (int)cdiv(p.N, BN);
  static const int gm = env_int("MLS_TILE_GM", 4);
  p.tile_gm = gm;
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles;
  hipLaunchKernelGGL((mfma16_w4_kernel<MT, OT, 256, BN, 2, 4, SPLIT>), dim3((unsigned)blocks), dim3(512), 0, st, p);
  return check_launch("INT4 GEMM");
}

template <int BKIND, typename MT, typename OT, int BM, int BN, int WM, int WN, bool GROUPED, bool SPLIT = false>
static int launch_adma(Mfma16Params p, hipStream_t st) {
  if constexpr (BKIND == B_INT8 && !GROUPED && BM == 256 && WM == 2 && WN == 4) {
    static const bool w8 = env_int("MLS_W8", 1) != 0;  // 0: the kernel above, for A/B runs
    if (w8) return launch_w8<MT, OT, BN, SPLIT>(p, st);

  }
  p.n_tiles = (int)cdiv(p.N, BN);
  const size_t lds = (size_t)2 * (BM + BN) * 8 * 16 + (BKIND == B_INT4 ? (size_t)2 * 2 * BN * 4 : 0);
  auto kern = mfma16_adma_kernel<BKIND, MT, OT, BM, BN, WM, WN, GROUPED, SPLIT>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(MLS_ERR_HIP, "mfma16 GEMM: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * WM * WN), lds, st, p);
  return check_launch("mfma16 GEMM");
}

// Two stages of register prefetch where the accumulators leave room for them: 8-wave
// blocks (two wavefronts per SIMD, 256 registers each) with at most 64 x 64 wave tiles.
template <int BM, int BN, int WM, int WN>
constexpr bool deep_prefetch() {
  return WM * WN == 8 && (BM / WM) * (BN / WN) <= 64 * 64;
}

template <int AKIND, int BKIND, typename MT, typename OT, int BM, int BN, int WM, int WN,
          bool GROUPED>
static int launch16(Mfma16Params p, hipStream_t st) {
  p.n_tiles = (int)cdiv(p.N, BN);
  const size_t lds = (size_t)2 * (BM + BN) * 8 * 16 + (BKIND == B_INT4 ? (size_t)2 * 2 * BN * 4 : 0);
  auto kern = mfma16_gemm_kernel<AKIND, BKIND, MT, OT, BM, BN, WM, WN, GROUPED,
                                 deep_prefetch<BM, BN, WM, WN>()>;
  static bool attr_set = false;  // raise the dynamic LDS limit once per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(MLS_ERR_HIP, "mfma16 GEMM: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * WM * WN), lds, st, p);
  return check_launch("mfma16 GEMM");
}

// Row-tile height for a dense GEMM: fewest (rounds of 256 blocks) x (BM + 128),
// where the 128 stands for the per-tile cost of staging and widening the B tile,
// which does not shrink with BM. Ties go to the taller tile.
static int pick_bm(int64_t M, int64_t N, int max_bm) {
  const int64_t nt = cdiv(N, 256);
  int best = 16;
  int64_t best_cost = INT64_MAX;
  for (int bm = 16; bm <= max_bm; bm *= 2) {
    if (bm > 16 && M <= bm / 2) break;
    const int64_t cost = cdiv(nt * cdiv(M, bm), 256) * (bm + 128);
    if (cost <= best_cost) {
      best_cost = cost;
      best = bm;
    }
  }
  return best;
}

// Tuning overrides for sweeps: MLS_BYTES = 0 keeps 256-row exact fp8 tiles on the kernel here
// instead of the byte-operand kernel (gemm_bytes.hip), MLS_MFMA_WAVES = 4 or 8 wavefronts per block (default 8:
// two per SIMD, so one wavefront's memory waits overlap the other's MFMAs), MLS_MFMA_BM =
// forced row-tile height (16 .. 256), MLS_MFMA_ADMA = 0 stages 16-bit activations
// through registers instead of loading them straight into LDS, MLS_MFMA_BN = 256 or 192
// forces the column-tile width of the 256-row weight-only kernel.

template <int AKIND, int BKIND, typename MT, typename OT>
static int dense16(Mfma16Params p, hipStream_t st) {
  constexpr int MAXBM = BKIND == B_INT4 ? 128 : 256;
  static const int waves = env_int("MLS_MFMA_WAVES", 8);
  static const int force_bm = env_int("MLS_MFMA_BM", 0);
  int bm = pick_bm(p.M, p.N, MAXBM);
  if (force_bm >= 16 && force_bm <= MAXBM && (force_bm & (force_bm - 1)) == 0) bm = force_bm;
  p.m_tiles = (int)cdiv(p.M, bm);
  const bool w8 = waves == 8;
  static const bool adma = env_int("MLS_MFMA_ADMA", 1) != 0;
  static const bool bytes = env_int("MLS_BYTES", 1) != 0;
  if (bytes && w8 && bm == 256) {
    if constexpr (AKIND != A_RAW16 && BKIND == B_E4M3)
      return launch_bytes_fp8(p, st, AKIND == A_E5M2,
                              __is_same(OT, float) ? MLS_F32 : __is_same(OT, _Float16) ? MLS_F16 : MLS_BF16);
  }
  if constexpr (AKIND == A_RAW16 && BKIND == B_INT4) {
    // 256 x 128 tiles on the INT4 kernel with the INT8 kernel's schedule, when they take no
    // more rounds of 256 blocks than the 128 x 256 tiles
    if (adma && w8 && w4_ok(p)) {
      const int64_t b_w4 = cdiv(p.M, 256) * cdiv(p.N, 128), b_128 = cdiv(p.M, 128) * cdiv(p.N, 256);
      if (cdiv(b_w4, 256) <= cdiv(b_128, 256)) return launch_w4<MT, OT>(p, st);
    }
  }
  if constexpr (AKIND == A_RAW16) {
    if (adma && w8 && bm == 256) {
      if constexpr (MAXBM >= 256) {
        // 256 x 192 tiles when fewer rounds of 256 blocks outweigh the smaller tile:
        // e.g. 2048 x 11008 is 344 blocks of 256 x 256 (two rounds, the second a
        // third full) but 464 blocks of 256 x 192 (two rounds, 25% less work each)
        static const int force_bn = env_int("MLS_MFMA_BN", 0);
        const int64_t mt = cdiv(p.M, 256);
        const int64_t c256 = cdiv(mt * cdiv(p.N, 256), 256) * 256, c192 = cdiv(mt * cdiv(p.N, 192), 256) * 192;
        if (force_bn == 192 || (force_bn != 256 && c192 < c256))
          return launch_adma<BKIND, MT, OT, 256, 192, 2, 4, false>(p, st);
        return launch_adma<BKIND, MT, OT, 256, 256, 2, 4, false>(p, st);
      }
    }
    if (adma && w8 && bm == 128) return launch_adma<BKIND, MT, OT, 128, 256, 2, 4, false>(p, st);
  }
  switch (bm) {
    case 256:
      if constexpr (MAXBM >= 256) {
        return w8 ? launch16<AKIND, BKIND, MT, OT, 256, 256, 2, 4, false>(p, st)
                  : launch16<AKIND, BKIND, MT, OT, 256, 256, 2, 2, false>(p, st);
      } else {
        return MLS_ERR_UNSUPPORTED;
      }
    case 128:
      return w8 ? launch16<AKIND, BKIND, MT, OT, 128, 256, 2, 4, false>(p, st)
                : launch16<AKIND, BKIND, MT, OT, 128, 256, 2, 2, false>(p, st);
    case 64: return launch16<AKIND, BKIND, MT, OT, 64, 256, 1, 4, false>(p, st);
    case 32: return launch16<AKIND, BKIND, MT, OT, 32, 256, 1, 4, false>(p, st);
    default: return launch16<AKIND, BKIND, MT, OT, 16, 256, 1, 4, false>(p, st);
  }
}

// One 256-row tile of each operand is addressed through a 32-bit buffer descriptor.
static bool tile_fits(int64_t a_row_bytes, int64_t b_row_bytes) {
  return a_row_bytes * 256 < (1ll << 31) && b_row_bytes * 256 < (1ll << 31);
}

int launch_gemm_wq_mfma(int wbits, const WqArgs& w) {
  if (w.a_dt != MLS_F16 && w.a_dt != MLS_BF16) return MLS_ERR_UNSUPPORTED;
  if (w.K % 64 != 0) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && w.group % 32 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.a, 16) || w.lda % 8 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.w, 16) || w.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.c, 8)) return MLS_ERR_UNSUPPORTED;
  if (w.M > 0x3FFFFFFF || w.N > 0x3FFFFFFF || w.K > 0x3FFFFFFF) return MLS_ERR_UNSUPPORTED;
  if (!tile_fits(w.lda * 2, w.ldw)) return MLS_ERR_UNSUPPORTED;
  Mfma16Params p{};
  p.a = w.a; p.lda = w.lda; p.b = w.w; p.ldb = w.ldw;
  p.s = w.s; p.s_dt = w.s_dt; p.ld_sn = w.ld_sn; p.ld_sg = w.ld_sg; p.group = w.group;
  p.c = w.c; p.ldc = w.ldc; p.M = (int)w.M; p.N = (int)w.N; p.K = (int)w.K;
  if (wbits == 4) {
    return w.a_dt == MLS_BF16 ? dense16<A_RAW16, B_INT4, __bf16, __bf16>(p, w.stream)
                              : dense16<A_RAW16, B_INT4, _Float16, _Float16>(p, w.stream);
  }
  return w.a_dt == MLS_BF16 ? dense16<A_RAW16, B_INT8, __bf16, __bf16>(p, w.stream)
                            : dense16<A_RAW16, B_INT8, _Float16, _Float16>(p, w.stream);
}

// The engine on split rows (fp32 activations as bf16 hi + lo, split.hip): w.a is the
// [split_rows(m_out)][lda] bf16 split matrix, w.M its row count, the output fp32 [m_out][ldc].
// 256-row tiles (INT8) or 128-row tiles; the epilogue adds each row's hi and lo products.
int launch_gemm_wq_mfma_split(int wbits, const WqArgs& w, int64_t m_out) {
  if (w.K % 64 != 0 || w.lda % 8 != 0 || !aligned(w.a, 16)) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && w.group % 32 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.w, 16) || w.ldw % 16 != 0 || !aligned(w.c, 8)) return MLS_ERR_UNSUPPORTED;
  if (w.M > 0x3FFFFFFF || w.N > 0x3FFFFFFF || w.K > 0x3FFFFFFF) return MLS_ERR_UNSUPPORTED;
  if (!tile_fits(w.lda * 2, w.ldw)) return MLS_ERR_UNSUPPORTED;
  Mfma16Params p{};
  p.a = w.a; p.lda = w.lda; p.b = w.w; p.ldb = w.ldw;
  p.s = w.s; p.s_dt = w.s_dt; p.ld_sn = w.ld_sn; p.ld_sg = w.ld_sg; p.group = w.group;
  p.c = w.c; p.ldc = w.ldc; p.M = (int)w.M; p.N = (int)w.N; p.K = (int)w.K;
  p.m_out = (int)m_out;
  if (wbits == 8 && w.M >= 256) {
    p.m_tiles = (int)cdiv(p.M, 256);
    const int64_t mt = p.m_tiles;
    const int64_t c256 = cdiv(mt * cdiv(p.N, 256), 256) * 256, c192 = cdiv(mt * cdiv(p.N, 192), 256) * 192;
    if (c192 < c256) return launch_adma<B_INT8, __bf16, float, 256, 192, 2, 4, false, true>(p, w.stream);
    return launch_adma<B_INT8, __bf16, float, 256, 256, 2, 4, false, true>(p, w.stream);
  }
  if (wbits == 4 && w4_ok(p) && cdiv(cdiv(p.M, 256) * cdiv(p.N, 128), 256) <= cdiv(cdiv(p.M, 128) * cdiv(p.N, 256), 256))
    return launch_w4<__bf16, float, true>(p, w.stream);
  p.m_tiles = (int)cdiv(p.M, 128);
  if (wbits == 8) return launch_adma<B_INT8, __bf16, float, 128, 256, 2, 4, false, true>(p, w.stream);
  return launch_adma<B_INT4, __bf16, float, 128, 256, 2, 4, false, true>(p, w.stream);
}

int launch_grouped_int4(const GroupedArgs& g) {
  const WqArgs& w = g.base;
  // gathered rows: offsets into a below the past-the-end offset of a missing row
  if (g.a_rows && (g.a_src_rows < 1 || g.a_src_rows * w.lda * 2 >= (1ll << 30))) return MLS_ERR_UNSUPPORTED;
  if (w.a_dt != MLS_F16 && w.a_dt != MLS_BF16) return MLS_ERR_UNSUPPORTED;
  if (w.K % 64 != 0 || w.group % 32 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.a, 16) || w.lda % 8 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.w, 16) || w.ldw % 16 != 0 || g.w_estride % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.c, 8)) return MLS_ERR_UNSUPPORTED;
  if (!tile_fits(w.lda * 2, w.ldw)) return MLS_ERR_UNSUPPORTED;
  constexpr int BM = 128;
  Mfma16Params p{};
  p.a = w.a; p.lda = w.lda; p.b = w.w; p.ldb = w.ldw;
  p.s = w.s; p.s_dt = w.s_dt; p.ld_sn = w.ld_sn; p.ld_sg = w.ld_sg; p.group = w.group;
  p.c = w.c; p.ldc = w.ldc; p.M = (int)w.M; p.N = (int)w.N; p.K = (int)w.K;
  p.seg_off = g.seg_off; p.E = g.E; p.b_estride = g.w_estride; p.s_estride = g.s_estride;
  p.a_rows = g.a_rows; p.a_src_rows = (int)g.a_src_rows;
  // MLS_GROUPED_TILES = 1: the row-tile kernels below instead of one block per expert
  // row chunk (gemm_grouped.hip)
  static const bool tiles = env_int("MLS_GROUPED_TILES", 0) != 0;
  if (!tiles || g.a_rows) return launch_grouped_seg(p, w.stream, w.a_dt == MLS_BF16, false);
  // upper bound on sum_e ceil(rows_e / BM) without reading the device offsets
  p.m_tiles = (int)(cdiv(w.M, BM) + g.E);
  static const bool w8 = env_int("MLS_MFMA_WAVES", 8) == 8;
  static const bool adma = env_int("MLS_MFMA_ADMA", 1) != 0;
  if (w8 && adma)
    return w.a_dt == MLS_BF16 ? launch_adma<B_INT4, __bf16, __bf16, BM, 256, 2, 4, true>(p, w.stream)
                              : launch_adma<B_INT4, _Float16, _Float16, BM, 256, 2, 4, true>(p, w.stream);
  if (w8)
    return w.a_dt == MLS_BF16 ? launch16<A_RAW16, B_INT4, __bf16, __bf16, BM, 256, 2, 4, true>(p, w.stream)
                              : launch16<A_RAW16, B_INT4, _Float16, _Float16, BM, 256, 2, 4, true>(p, w.stream);
  return w.a_dt == MLS_BF16 ? launch16<A_RAW16, B_INT4, __bf16, __bf16, BM, 256, 2, 2, true>(p, w.stream)
                            : launch16<A_RAW16, B_INT4, _Float16, _Float16, BM, 256, 2, 2, true>(p, w.stream);
}

int launch_grouped_gate_up(const GroupedArgs& g, const uint8_t* wu, const void* su) {
  const WqArgs& w = g.base;
  // gathered rows: offsets into a below the past-the-end offset of a missing row
  if (g.a_rows && (g.a_src_rows < 1 || g.a_src_rows * w.lda * 2 >= (1ll << 30))) return MLS_ERR_UNSUPPORTED;
  if (w.a_dt != MLS_F16 && w.a_dt != MLS_BF16) return MLS_ERR_UNSUPPORTED;
  if (w.K % 64 != 0 || w.group % 32 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.a, 16) || w.lda % 8 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.w, 16) || !aligned(wu, 16) || w.ldw % 16 != 0 || g.w_estride % 16 != 0)
    return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.c, 8) || !tile_fits(w.lda * 2, w.ldw)) return MLS_ERR_UNSUPPORTED;
  Mfma16Params p{};
  p.a = w.a; p.lda = w.lda; p.b = w.w; p.ldb = w.ldw; p.b2 = wu;
  p.s = w.s; p.s2 = su; p.s_dt = w.s_dt; p.ld_sn = w.ld_sn; p.ld_sg = w.ld_sg; p.group = w.group;
  p.c = w.c; p.ldc = w.ldc; p.M = (int)w.M; p.N = (int)w.N; p.K = (int)w.K;
  p.seg_off = g.seg_off; p.E = g.E; p.b_estride = g.w_estride; p.s_estride = g.s_estride;
  p.a_rows = g.a_rows; p.a_src_rows = (int)g.a_src_rows;
  return launch_grouped_seg(p, w.stream, w.a_dt == MLS_BF16, true);
}

int launch_grouped_int4_partial(const GroupedArgs& g, int splits, float* partial, int64_t ldp, int64_t sstride) {
  const WqArgs& w = g.base;
  if (w.a_dt != MLS_F16 && w.a_dt != MLS_BF16) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.a, 16) || w.lda % 8 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(w.w, 16) || w.ldw % 16 != 0 || g.w_estride % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(partial, 16) || !tile_fits(w.lda * 2, w.ldw)) return MLS_ERR_UNSUPPORTED;
  Mfma16Params p{};
  p.a = w.a; p.lda = w.lda; p.b = w.w; p.ldb = w.ldw;
  p.s = w.s; p.s_dt = w.s_dt; p.ld_sn = w.ld_sn; p.ld_sg = w.ld_sg; p.group = w.group;
  p.c = partial; p.ldc = ldp; p.M = (int)w.M; p.N = (int)w.N; p.K = (int)w.K;
  p.seg_off = g.seg_off; p.E = g.E; p.b_estride = g.w_estride; p.s_estride = g.s_estride;
  p.a_rows = g.a_rows; p.a_src_rows = (int)g.a_src_rows;
  p.ksplit = splits; p.c_sstride = sstride;
  return launch_grouped_partial(p, w.stream, w.a_dt == MLS_BF16);
}

int launch_fp8_exact(const Fp8Args& f) {
  if (f.K % 64 != 0 || f.M < 16 || f.N < 16) return MLS_ERR_UNSUPPORTED;
  if (!aligned(f.a, 16) || !aligned(f.b, 16) || f.lda % 16 != 0 || f.ldb % 16 != 0)
    return MLS_ERR_UNSUPPORTED;
  if (!aligned(f.c, 16) || !tile_fits(f.lda, f.ldb)) return MLS_ERR_UNSUPPORTED;
  if (f.M > 0x3FFFFFFF || f.N > 0x3FFFFFFF || f.K > 0x3FFFFFFF) return MLS_ERR_UNSUPPORTED;
  Mfma16Params p{};
  p.a = f.a; p.lda = f.lda; p.b = f.b; p.ldb = f.ldb;
  p.sa = f.sa; p.sap = f.sap; p.sas = f.sas; p.sb = f.sb; p.sbp = f.sbp; p.sbs = f.sbs;
  p.c = f.c; p.ldc = f.ldc; p.M = (int)f.M; p.N = (int)f.N; p.K = (int)f.K;
  if (f.a_e5m2) {
    if (f.c_dt == MLS_F32) return dense16<A_E5M2, B_E4M3, __bf16, float>(p, f.stream);
    if (f.c_dt == MLS_F16) return dense16<A_E5M2, B_E4M3, __bf16, _Float16>(p, f.stream);
    return dense16<A_E5M2, B_E4M3, __bf16, __bf16>(p, f.stream);
  }
  if (f.c_dt == MLS_F32) return dense16<A_E4M3, B_E4M3, __bf16, float>(p, f.stream);
  if (f.c_dt == MLS_F16) return dense16<A_E4M3, B_E4M3, __bf16, _Float16>(p, f.stream);
  return dense16<A_E4M3, B_E4M3, __bf16, __bf16>(p, f.stream);
}

}  // namespace mls
