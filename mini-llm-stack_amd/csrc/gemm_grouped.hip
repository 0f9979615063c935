// Grouped (per-expert) INT4 weight-only GEMM for MoE: one launch over every expert's
// row segment, segment offsets read on the device.
//
// A block owns one expert's row chunk (up to BMX = 32 TMX rows of its segment; a
// segment longer than BMX is split into chunks) and 128 weight rows n, and streams K
// in 64-k stages. So each weight byte is read and widened once per row chunk (once per
// expert when the segment fits in one chunk, as in config E: 115-136 rows per expert),
// and only the 16-row subtiles that hold segment rows are multiplied.
//
// 4 wavefronts as 2 (m) x 2 (n): wavefront (wm, wn) owns columns 64 wn .. 64 wn + 63
// and the 16-row subtiles 2 t + wm (t < TMX) that the chunk covers. 256 threads and
// ~72 KiB of LDS per block, so two blocks share a CU.
//
// Per stage (LDS buffer kt & 1): store stage kt + 1's widened weights, read this
// stage's operands, issue stage kt + 1's activation rows straight into LDS
// (buffer_load ... lds), then the weight loads of stage kt + 3, MFMAs
// (v_mfma_f32_16x16x32), and a barrier that waits only for the LDS-direct loads
// (vmcnt(1): the weight load issued after them stays in flight; a __syncthreads()
// would drain it too and expose the full HBM latency every stage). LDS rows are 64 k = 128 bytes, 16-byte chunk
// index XOR row & 7 (conflict-free for these 16-row operand reads and chunk stores).
//
// INT4 widening, exact, 16 VALU per 8 weights: x = d ^ 0x88888888 turns each nibble
// v into v ^ 8; masking the high nibbles (x & 0xF0F0F0F0) and the shifted low nibbles
// ((x << 4) & 0xF0F0F0F0) leaves bytes whose signed value is 16 (v - 8); a sign-
// extending SDWA convert per byte gives the exact float, and the 1/16 is folded into
// the group scale (a power of two: exact). Group scales apply to fp32 partial sums at
// every group boundary, as in the dense INT4 kernels.
#include "mfma16.h"

namespace mls {

namespace {

// 32 INT4 weights (16 bytes, even k in the low nibble) -> 16 dwords of 16-bit floats
// holding 16 (v - 8), k order.
template <typename MT>
__device__ __forceinline__ void widen_int4x16(const uint4& q, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t x = d[t] ^ 0x88888888u;
    const uint32_t hi = x & 0xF0F0F0F0u;         // k = 8t + 1, 3, 5, 7 (byte b: k = 8t + 2b + 1)
    const uint32_t lo = (x << 4) & 0xF0F0F0F0u;  // k = 8t + 0, 2, 4, 6
    o[4 * t + 0] = pack_exact2<MT>(sbyte_f32<0>(lo), sbyte_f32<0>(hi));
    o[4 * t + 1] = pack_exact2<MT>(sbyte_f32<1>(lo), sbyte_f32<1>(hi));
    o[4 * t + 2] = pack_exact2<MT>(sbyte_f32<2>(lo), sbyte_f32<2>(hi));
    o[4 * t + 3] = pack_exact2<MT>(sbyte_f32<3>(lo), sbyte_f32<3>(hi));
  }
}

}  // namespace

// STAB: the block's whole [128 x G] fp16 group-scale table is loaded once, coalesced,
// into LDS (G <= 32, contiguous groups). Otherwise each stage loads the scales of its
// 128 rows; those loads touch one cache line per row, many more L2 requests than the
// weights themselves, and their latency then dominates the stage.
// GU (gate/up of a SwiGLU expert MLP): the block's 128 weight rows are 64 rows of the
// gate matrix (p.b, p.s) and the same 64 rows of the up matrix (p.b2, p.s2); the
// epilogue writes h = silu(gate) * up for those 64 columns, from the fp32 accumulators.
template <typename MT, typename OT, int TMX, bool STAB, bool GU>
__global__ __launch_bounds__(256, 2) void grouped_int4_kernel(const Mfma16Params p) {
  constexpr int BN = 128, BK = 64, NT = 256;
  constexpr int OUTN = GU ? 64 : 128;  // output columns per block
  constexpr int BMX = 32 * TMX, TN = 4;
  constexpr int PW = BMX * 8 / NT;  // activation LDS-direct loads per thread and stage
  static_assert(BMX * 8 % NT == 0, "activation slots");

  extern __shared__ __align__(16) uint8_t smem[];
  uint4* As = reinterpret_cast<uint4*>(smem);             // [2][BMX][8]
  uint4* Bs = As + 2 * BMX * 8;                            // [2][BN][8]
  float* sS = reinterpret_cast<float*>(Bs + 2 * BN * 8);  // [2][2][BN] (per-stage scales)
  _Float16* sT = reinterpret_cast<_Float16*>(Bs + 2 * BN * 8);  // [G][BN] (STAB)

  // ---- which (expert, row chunk, column tile). The grid is sized by a bound on the
  // row chunks; the blocks past the real item count exit, and the real items are
  // spread over the XCDs by their own count (remapping over the whole grid would park
  // every surplus block on the last XCDs and leave them idle). Consecutive logical ids
  // share the row chunk and sit on one XCD.
  int chunks = 0;
  for (int e = 0; e < p.E; ++e) chunks += (p.seg_off[e + 1] - p.seg_off[e] + BMX - 1) / BMX;
  const int items = chunks * p.n_tiles;
  if ((int)blockIdx.x >= items) return;
  const int L = xcd_remap(blockIdx.x, items);
  const int chunk = L / p.n_tiles, nt = L % p.n_tiles;
  int e = 0, cum = 0, lo = 0, hi = 0;
  for (; e < p.E; ++e) {
    lo = p.seg_off[e];
    hi = p.seg_off[e + 1];
    const int t = (hi - lo + BMX - 1) / BMX;
    if (chunk < cum + t) break;
    cum += t;
  }
  const int m0 = __builtin_amdgcn_readfirstlane(lo + (chunk - cum) * BMX);
  const int rows = __builtin_amdgcn_readfirstlane(min(BMX, hi - m0));
  const int nsub = (rows + 15) >> 4;  // active 16-row subtiles
  const int ssz = p.s_dt == MLS_F16 ? 2 : 4;
  const uint8_t* bmat = p.b + (int64_t)e * p.b_estride;
  const uint8_t* smat = (const uint8_t*)p.s + (int64_t)e * p.s_estride * ssz;
  const int n0 = nt * OUTN, N = p.N;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lk = lane >> 4;
  if constexpr (GU) {
    // waves 2 and 3 stage B rows 64 .. 127: the up matrix
    if (wave >= 2) bmat = p.b2 + (int64_t)e * p.b_estride;
  }
  const uint8_t* smat_hi = GU ? (const uint8_t*)p.s2 + (int64_t)e * p.s_estride * ssz : smat;

  const int rows_b = __builtin_amdgcn_readfirstlane(min(OUTN, N - n0));
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + (int64_t)m0 * p.lda * 2), (short)0, (int)(rows * p.lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(bmat + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb), 0x00020000);
  // activation slot t = (wave * PW + i) * 64 + lane: row t / 8, logical chunk (t % 8) ^ (row & 7)
  int a_off[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int t = (wave * PW + i) * 64 + lane, row = t >> 3, lc = (t & 7) ^ (row & 7);
    a_off[i] = row * (int)p.lda * 2 + lc * 16;
  }
  // weights: thread tid stages B row tid / 2 (GU: row (tid / 2) % 64 of its matrix),
  // 16-byte column tid % 2 (32 k) of the stage
  const int b_row = tid >> 1, b_cc = tid & 1;
  const int b_off = (GU ? (b_row & 63) : b_row) * (int)p.ldb + b_cc * 16;
  const int s_r = tid & (BN - 1);  // B row whose per-stage scales this thread loads
  const uint8_t* s_mat = (GU && s_r >= 64) ? smat_hi : smat;
  const int64_t s_row = (int64_t)min(n0 + (GU ? (s_r & 63) : s_r), N - 1) * p.ld_sn;

  // weights of the stage to store next (rb, rs0, rs1) and of the one after (nb, ns0, ns1)
  uint4 rb, nb;
  float rs0 = 0.f, rs1 = 0.f, ns0 = 0.f, ns1 = 0.f;
  auto dma_a = [&](int buf, int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PW; ++i) lds_load16(rsa, As + buf * BMX * 8 + (wave * PW + i) * 64, a_off[i], k0 * 2);
  };
  // the weight chunk first, then (per-stage scales) the scale loads; threads past BN
  // re-read a scale they never store
  auto load_b = [&](int k0, uint4& w, float& s0, float& s1) __attribute__((always_inline)) {
    w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsb, b_off, k0 / 2, 0));
    if constexpr (!STAB) {
      const int kc = min(k0, p.K - BK);  // a stage past the end reuses the last scales
      s0 = scale_at(s_mat, p.s_dt, s_row + (int64_t)(kc / p.group) * p.ld_sg) * 0.0625f;
      s1 = scale_at(s_mat, p.s_dt, s_row + (int64_t)((kc + 32) / p.group) * p.ld_sg) * 0.0625f;
    }
  };
  auto store_b = [&](int buf) __attribute__((always_inline)) {
    uint4* bs = Bs + buf * BN * 8;
    uint32_t o[16];
    widen_int4x16<MT>(rb, o);
#pragma unroll
    for (int h = 0; h < 4; ++h)
      bs[b_row * 8 + ((4 * b_cc + h) ^ swz(b_row))] = make_uint4(o[4 * h + 0], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
    if (!STAB && tid < BN) {
      sS[(buf * 2 + 0) * BN + tid] = rs0;
      sS[(buf * 2 + 1) * BN + tid] = rs1;
    }
  };

  f32x4 acc[TN][TMX], accg[TN][TMX];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TMX; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const int nk = p.K / BK;
  if constexpr (STAB) {
    // scale table: row n0 + r holds G fp16 scales; 16-byte piece c = tid + 256 i is
    // row c / (G / 8), groups 8 (c % (G / 8)) .. + 7, written transposed to sT[g][r]
    const int G = p.K / p.group, ppr = G / 8;
    for (int c = tid; c < BN * ppr; c += 256) {
      const int r = c / ppr, part = c % ppr;
      const int64_t n = min(n0 + (GU ? (r & 63) : r), N - 1);
      const uint8_t* sm = (GU && r >= 64) ? smat_hi : smat;
      const uint4 v = *reinterpret_cast<const uint4*>((const _Float16*)sm + n * p.ld_sn + part * 8);
      const _Float16* h = reinterpret_cast<const _Float16*>(&v);
#pragma unroll
      for (int t = 0; t < 8; ++t) sT[(part * 8 + t) * BN + r] = h[t];
    }
  }
  // prologue: stage 0 into buffer 0; stages 1 and 2 in registers
  dma_a(0, 0);
  load_b(0, rb, rs0, rs1);
  __builtin_amdgcn_s_waitcnt(0);
  store_b(0);
  load_b(BK, rb, rs0, rs1);
  load_b(2 * BK, nb, ns0, ns1);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const int k0 = kt * BK;
    store_b(buf ^ 1);  // stage kt + 1 (past the end: harmless)
    const uint4* as = As + buf * BMX * 8;
    const uint4* bs = Bs + buf * BN * 8;
    // one 32-k half at a time (operand registers for one half only); the next stage's
    // LDS-direct loads go out after the last operand read of this stage, so the wait
    // the compiler keeps before LDS reads behind them falls on the barrier
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 aop[TMX], bop[TN];
      const int ch = ks * 4 + lk;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int row = wn * 64 + i * 16 + lr;
        bop[i] = bs[row * 8 + (ch ^ swz(row))];
      }
#pragma unroll
      for (int j = 0; j < TMX; ++j) {
        const int row = (2 * j + wm) * 16 + lr;
        aop[j] = as[row * 8 + (ch ^ swz(row))];
      }
      float sc[TN][4];
      if constexpr (STAB) {
        const int g = (k0 + 32 * ks) / p.group;
#pragma unroll
        for (int i = 0; i < TN; ++i) {
          const uint2 h2 = *reinterpret_cast<const uint2*>(sT + g * BN + wn * 64 + i * 16 + 4 * lk);
          const _Float16* h = reinterpret_cast<const _Float16*>(&h2);
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[i][r] = (float)h[r] * 0.0625f;
        }
      } else {
#pragma unroll
        for (int i = 0; i < TN; ++i) {
          const float4 s4 = *reinterpret_cast<const float4*>(sS + (buf * 2 + ks) * BN + wn * 64 + i * 16 + 4 * lk);
          sc[i][0] = s4.x;
          sc[i][1] = s4.y;
          sc[i][2] = s4.z;
          sc[i][3] = s4.w;
        }
      }
      if (ks == 1) {
        __builtin_amdgcn_sched_barrier(0);
        dma_a(buf ^ 1, k0 + BK);  // stage kt + 1 (past the end: zeros / harmless)
        // the weight loads must issue after the LDS-direct loads: the vmcnt(1) before
        // the barrier counts on the LDS-direct loads being the older ones
        __builtin_amdgcn_sched_barrier(0);
        // stage kt + 2's weights move up (loaded during stage kt - 1), stage kt + 3's go out
        rb = nb;
        rs0 = ns0;
        rs1 = ns1;
        load_b(k0 + 3 * BK, nb, ns0, ns1);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < TMX; ++j) {
        if (2 * j + wm >= nsub) continue;  // subtile past the segment: nothing to multiply
#pragma unroll
        for (int i = 0; i < TN; ++i) accg[i][j] = Mfma16<MT>::mma(bop[i], aop[j], accg[i][j]);
      }
      if ((k0 + 32 * (ks + 1)) % p.group == 0) {  // group ends: acc += s[n] * partial
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TMX; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(sc[i][r], accg[i][j][r], acc[i][j][r]);
            accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    // every wavefront's LDS-direct loads of stage kt + 1 and LDS stores land before the
    // barrier. At least one load (the weight chunk) is issued after the LDS-direct loads
    // and loads complete in order, so vmcnt(1) covers them whatever number of scale
    // loads follows; the last weight load stays in flight
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- epilogue: acc[i][j][r] = C[m = m0 + (2 j + wm) 16 + lr][n = n0 + 64 wn + 16 i + 4 lk + r]
  OT* c = static_cast<OT*>(p.c);
  if constexpr (GU) {
    // wavefronts wn = 1 hold the up products: they pass them through LDS (the
    // activation buffers, free after the loop's last barrier) to the wavefronts wn = 0,
    // which hold the gate products of the same (m, n) and write silu(gate) * up
    float* U = reinterpret_cast<float*>(smem);  // [BMX][64]
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TMX; ++j)
          *reinterpret_cast<f32x4*>(U + ((2 * j + wm) * 16 + lr) * 64 + i * 16 + 4 * lk) = acc[i][j];
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (wn == 1) return;
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int nb = n0 + i * 16 + 4 * lk;
#pragma unroll
      for (int j = 0; j < TMX; ++j) {
        const int ml = (2 * j + wm) * 16 + lr;
        if (ml >= rows) continue;
        const f32x4 u = *reinterpret_cast<const f32x4*>(U + ml * 64 + i * 16 + 4 * lk);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float g = acc[i][j][r];
          v[r] = g / (1.0f + __expf(-g)) * u[r];
        }
        OT* dst = c + (int64_t)(m0 + ml) * p.ldc + nb;
        if (nb + 3 < N && (p.ldc % 4) == 0) {
          store4<OT>(dst, v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nb + r < N) dst[r] = from_f32<OT>(v[r]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn * 64 + i * 16 + 4 * lk;
#pragma unroll
    for (int j = 0; j < TMX; ++j) {
      const int ml = (2 * j + wm) * 16 + lr;
      if (ml >= rows) continue;
      OT* dst = c + (int64_t)(m0 + ml) * p.ldc + nb;
      if (nb + 3 < N && (p.ldc % 4) == 0) {
        store4<OT>(dst, acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) dst[r] = from_f32<OT>(acc[i][j][r]);
      }
    }
  }
}

template <typename MT, int TMX, bool STAB, bool GU>
static int launch_grouped(Mfma16Params p, hipStream_t st) {
  constexpr int BMX = 32 * TMX, BN = 128, OUTN = GU ? 64 : 128;
  p.n_tiles = (int)cdiv(p.N, OUTN);
  // upper bound on sum_e ceil(rows_e / BMX) without reading the device offsets
  p.m_tiles = (int)(cdiv(p.M, BMX) + p.E);
  const size_t tab = STAB ? (size_t)BN * 32 * 2 : (size_t)2 * 2 * BN * 4;
  const size_t lds = (size_t)2 * (BMX + BN) * 8 * 16 + tab;
  auto kern = grouped_int4_kernel<MT, MT, TMX, STAB, GU>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(MLS_ERR_HIP, "grouped INT4 GEMM: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles;
  if (blocks > 0x7FFFFFFF) return MLS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), lds, st, p);
  return check_launch(GU ? "grouped INT4 gate/up GEMM" : "grouped INT4 GEMM");
}

template <bool STAB, bool GU>
static int launch_grouped_tmx(const Mfma16Params& p, hipStream_t st, bool bf16, int tmx) {
  switch (tmx) {
    case 5: return bf16 ? launch_grouped<__bf16, 5, STAB, GU>(p, st) : launch_grouped<_Float16, 5, STAB, GU>(p, st);
    case 4: return bf16 ? launch_grouped<__bf16, 4, STAB, GU>(p, st) : launch_grouped<_Float16, 4, STAB, GU>(p, st);
    case 3: return bf16 ? launch_grouped<__bf16, 3, STAB, GU>(p, st) : launch_grouped<_Float16, 3, STAB, GU>(p, st);
    default: return bf16 ? launch_grouped<__bf16, 2, STAB, GU>(p, st) : launch_grouped<_Float16, 2, STAB, GU>(p, st);
  }
}

// Row-chunk height: the smallest of 64 / 96 / 128 / 160 rows that holds 1.25x the
// average segment (routed segments scatter around the average), so a typical expert's
// rows fit in one chunk and its weights are streamed and widened once.
int launch_grouped_seg(const Mfma16Params& p, hipStream_t st, bool bf16, bool gate_up) {
  const int64_t want = cdiv(p.M * 5, p.E * 4);
  const int tmx = want > 128 ? 5 : want > 96 ? 4 : want > 64 ? 3 : 2;
  // scale table in LDS: fp16 scales, contiguous groups, G a multiple of 8 up to 32,
  // 16-byte aligned rows
  const int64_t G = p.K / p.group;
  const bool stab = p.s_dt == MLS_F16 && p.ld_sg == 1 && G % 8 == 0 && G <= 32 && (p.ld_sn % 8) == 0 &&
                    (p.s_estride % 8) == 0 && aligned(p.s, 16) && (!gate_up || aligned(p.s2, 16));
  if (gate_up)
    return stab ? launch_grouped_tmx<true, true>(p, st, bf16, tmx) : launch_grouped_tmx<false, true>(p, st, bf16, tmx);
  return stab ? launch_grouped_tmx<true, false>(p, st, bf16, tmx) : launch_grouped_tmx<false, false>(p, st, bf16, tmx);
}

}  // namespace mls
