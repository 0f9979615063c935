// Grouped (per-expert) INT4 weight-only GEMM for MoE: one launch over every expert's
// row segment, segment offsets read on the device.
//
// A block owns one expert's row chunk (up to BMX = 32 TMX rows of its segment; a
// segment longer than BMX is split into chunks) and 128 weight rows n, and streams K
// in 64-k stages. So each weight byte is read and widened once per row chunk (once per
// expert when the segment fits in one chunk, as in config E: 115-136 rows per expert).
// Rows of the chunk past the segment are zeros and are multiplied too (branch-free).
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
// extending SDWA convert per byte gives the exact float, and the 1/16 (a power of two:
// exact) is applied once to the results. Group scales apply to fp32 partial sums at
// every group boundary, as in the dense INT4 kernels, and are read only there.
#include <type_traits>

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
// into LDS (G <= 128 and a multiple of 4, contiguous groups: at most 32 KiB).
// Otherwise each stage loads the
// scales of its 128 rows; those loads touch one cache line per row, many more L2
// requests than the weights themselves. They are issued before the stage's LDS-direct
// activation loads, so the end-of-stage wait, which must cover the LDS-direct loads,
// leaves only the weight load in flight behind them.
// GU (gate/up of a SwiGLU expert MLP): the block's 128 weight rows are 64 rows of the
// gate matrix (p.b, p.s) and the same 64 rows of the up matrix (p.b2, p.s2); the
// epilogue writes h = silu(gate) * up for those 64 columns, from the fp32 accumulators.
// offset of a gathered activation row that is not there: past any descriptor's range
// (below 2^31 even with the stage's k offset added)
constexpr int kPastEndA = 0x40000000;

template <int R>
struct Ring {
  static constexpr int v = R;
};

// SCL: 32 or 128 = fp16 scale table of up to that many groups (STAB); 0 / 1 = fp32 /
// fp16 scales loaded per stage (the dtype fixed at compile time, so the loaded values
// are not consumed, and waited for, until they are stored two stages later).
template <typename MT, typename OT, int TMX, int SCL, bool GU>
__global__ __launch_bounds__(256, 2) void grouped_int4_kernel(const Mfma16Params p) {
  constexpr bool STAB = SCL >= 32;
  constexpr int TABG = STAB ? SCL : 0;
  constexpr int BN = 128, BK = 64, NT = 256;
  constexpr int OUTN = GU ? 64 : 128;  // output columns per block
  constexpr int BMX = 32 * TMX, TN = 4;
  constexpr int PW = BMX * 8 / NT;  // activation LDS-direct loads per thread and stage
  static_assert(BMX * 8 % NT == 0, "activation slots");

  // Double-buffered activation and widened-weight tiles in separate arrays: the
  // compiler then knows that a pending LDS-direct load into one buffer cannot touch
  // the other (or the scale table), and inserts no wait for it before their reads.
  // 72 KiB at TMX = 5; with a scale table of up to 32 groups (8 KiB) two blocks share
  // a CU.
  __shared__ __align__(16) uint4 As0[BMX * 8], As1[BMX * 8];
  __shared__ __align__(16) uint4 Bs0[BN * 8], Bs1[BN * 8];
  __shared__ __align__(16) uint8_t sTab[STAB ? TABG * BN * 2 : 2 * 2 * BN * 4];
  _Float16* const sT = reinterpret_cast<_Float16*>(sTab);  // [G][BN] fp16 (STAB)
  float* const sS = reinterpret_cast<float*>(sTab);        // [2][2][BN] per-stage scales

  // ---- which (expert, row chunk, column tile). The grid is sized by a bound on the
  // row chunks; the blocks past the real item count exit, and the real items are
  // spread over the XCDs by their own count (remapping over the whole grid would park
  // every surplus block on the last XCDs and leave them idle). Consecutive logical ids
  // share the row chunk and sit on one XCD.
  // With a K split, item = (chunk, split, column tile): the splits of one chunk sit on
  // one XCD next to its column tiles, sharing the chunk's activation rows in L2.
  const int ksn = p.ksplit > 1 ? p.ksplit : 1;
  int chunks = 0;
  for (int e = 0; e < p.E; ++e) {
    int lo, hi;
    seg_rows(p, e, lo, hi);
    chunks += (hi - lo + BMX - 1) / BMX;
  }
  const int items = chunks * p.n_tiles * ksn;
  if ((int)blockIdx.x >= items) return;
  const int L = xcd_remap(blockIdx.x, items);
  const int chunk = L / (p.n_tiles * ksn), rem = L % (p.n_tiles * ksn);
  const int split = rem / p.n_tiles, nt = rem % p.n_tiles;
  const int Kp = p.K / ksn, kbase = split * Kp;  // this block's K range
  int e = 0, cum = 0, lo = 0, hi = 0;
  for (; e < p.E; ++e) {
    seg_rows(p, e, lo, hi);
    const int t = (hi - lo + BMX - 1) / BMX;
    if (chunk < cum + t) break;
    cum += t;
  }
  const int m0 = __builtin_amdgcn_readfirstlane(lo + (chunk - cum) * BMX);
  const int rows = __builtin_amdgcn_readfirstlane(min(BMX, hi - m0));
  constexpr int ssz = SCL == 0 ? 4 : 2;
  const uint8_t* bmat = p.b + (int64_t)e * p.b_estride + kbase / 2;
  const uint8_t* smat = (const uint8_t*)p.s + ((int64_t)e * p.s_estride + (int64_t)(kbase / p.group) * p.ld_sg) * ssz;
  const int n0 = nt * OUTN, N = p.N;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lk = lane >> 4;
  if constexpr (GU) {
    // waves 2 and 3 stage B rows 64 .. 127: the up matrix
    if (wave >= 2) bmat = p.b2 + (int64_t)e * p.b_estride + kbase / 2;
  }
  const uint8_t* smat_hi =
      GU ? (const uint8_t*)p.s2 + ((int64_t)e * p.s_estride + (int64_t)(kbase / p.group) * p.ld_sg) * ssz : smat;

  const int rows_b = __builtin_amdgcn_readfirstlane(min(OUTN, N - n0));
  // activations: the chunk's rows m0 .. m0 + rows - 1 of a, or with a_rows (the dispatch
  // gather fused into the load) rows a_rows[m0 + r] of a; rows past the chunk, and source
  // rows outside a, read zeros
  const bool gather = p.a_rows != nullptr;
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + ((gather ? 0 : (int64_t)m0 * p.lda) + kbase) * 2), (short)0,
      (int)((gather ? p.a_src_rows : rows) * p.lda * 2 - kbase * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(bmat + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb - kbase / 2), 0x00020000);
  // activation slot t = (wave * PW + i) * 64 + lane: row t / 8, logical chunk (t % 8) ^ (row & 7)
  int a_off[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int t = (wave * PW + i) * 64 + lane, row = t >> 3, lc = (t & 7) ^ (row & 7);
    if (gather) {
      const int src = row < rows ? p.a_rows[m0 + row] : -1;
      a_off[i] = (src >= 0 && src < p.a_src_rows) ? src * (int)p.lda * 2 + lc * 16 : kPastEndA;
    } else {
      a_off[i] = row * (int)p.lda * 2 + lc * 16;
    }
  }
  // weights: thread tid stages B row tid / 2 (GU: row (tid / 2) % 64 of its matrix),
  // 16-byte column tid % 2 (32 k) of the stage
  const int b_row = tid >> 1, b_cc = tid & 1;
  const int b_off = (GU ? (b_row & 63) : b_row) * (int)p.ldb + b_cc * 16;
  const int s_r = tid & (BN - 1);  // B row whose per-stage scales this thread loads
  const uint8_t* s_mat = (GU && s_r >= 64) ? smat_hi : smat;
  const int64_t s_row = (int64_t)min(n0 + (GU ? (s_r & 63) : s_r), N - 1) * p.ld_sn;

  auto abuf = [&](auto r) __attribute__((always_inline)) -> uint4* {
    if constexpr (decltype(r)::v == 0) return As0;
    else return As1;
  };
  auto bbuf = [&](auto r) __attribute__((always_inline)) -> uint4* {
    if constexpr (decltype(r)::v == 0) return Bs0;
    else return Bs1;
  };

  // weight chunks (and per-stage scales) in a register ring of three: slot kt % 3 holds
  // stage kt's chunk until it is stored (stage kt - 1), then receives stage kt + 3's.
  // The slots are named variables selected at compile time, so no register copies
  // (each of which would wait for its load) sit between a load and its use.
  uint4 w0, w1, w2;
  float s00 = 0.f, s01 = 0.f, s10 = 0.f, s11 = 0.f, s20 = 0.f, s21 = 0.f;
  auto wreg = [&](auto q) __attribute__((always_inline)) -> uint4& {
    if constexpr (decltype(q)::v == 0) return w0;
    else if constexpr (decltype(q)::v == 1) return w1;
    else return w2;
  };
  auto sreg0 = [&](auto q) __attribute__((always_inline)) -> float& {
    if constexpr (decltype(q)::v == 0) return s00;
    else if constexpr (decltype(q)::v == 1) return s10;
    else return s20;
  };
  auto sreg1 = [&](auto q) __attribute__((always_inline)) -> float& {
    if constexpr (decltype(q)::v == 0) return s01;
    else if constexpr (decltype(q)::v == 1) return s11;
    else return s21;
  };
  auto dma_a = [&](uint4* dst, int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PW; ++i) lds_load16(rsa, dst + (wave * PW + i) * 64, a_off[i], k0 * 2);
  };
  // per-stage scales (!STAB); threads past BN re-read a scale they never store
  auto load_s = [&](int k0, float& s0, float& s1) __attribute__((always_inline)) {
    if constexpr (!STAB) {
      const int kc = min(k0, Kp - BK);  // a stage past the end reuses the last scales
      using ST = std::conditional_t<SCL == 1, _Float16, float>;
      const ST* sp = reinterpret_cast<const ST*>(s_mat) + s_row;
      s0 = (float)sp[(int64_t)(kc / p.group) * p.ld_sg];
      s1 = (float)sp[(int64_t)((kc + 32) / p.group) * p.ld_sg];
    }
  };
  auto load_w = [&](int k0, uint4& w) __attribute__((always_inline)) {
    w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsb, b_off, k0 / 2, 0));
  };
  auto store_b = [&](auto r, const uint4& w, float t0, float t1) __attribute__((always_inline)) {
    uint4* bs = bbuf(r);
    uint32_t o[16];
    widen_int4x16<MT>(w, o);
#pragma unroll
    for (int h = 0; h < 4; ++h)
      bs[b_row * 8 + ((4 * b_cc + h) ^ swz(b_row))] = make_uint4(o[4 * h + 0], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
    if (!STAB && tid < BN) {
      sS[(decltype(r)::v * 2 + 0) * BN + tid] = t0;
      sS[(decltype(r)::v * 2 + 1) * BN + tid] = t1;
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

  const int nk = Kp / BK;
  const int G_blk = Kp / p.group;  // groups of this block's K range
  if constexpr (STAB) {
    // scale table: row n0 + r holds G fp16 scales; 16-byte piece c = tid + 256 i is
    // row c / (G / 8), groups 8 (c % (G / 8)) .. + 7, written transposed to sT[g][r]
    const int G = Kp / p.group, ppr = G / 4;
    for (int c = tid; c < BN * ppr; c += 256) {
      const int r = c / ppr, part = c % ppr;
      const int64_t n = min(n0 + (GU ? (r & 63) : r), N - 1);
      const uint8_t* sm = (GU && r >= 64) ? smat_hi : smat;
      const uint2 v = *reinterpret_cast<const uint2*>((const _Float16*)sm + n * p.ld_sn + part * 4);
      const _Float16* h = reinterpret_cast<const _Float16*>(&v);
#pragma unroll
      for (int t = 0; t < 4; ++t) sT[(part * 4 + t) * BN + r] = h[t];
    }
  }

  // Stage kt on LDS buffer r = kt % 2 and register slot q = kt % 3. At its start (the
  // buffers r ^ 1 were last read in stage kt - 1, before the barrier that ended it):
  // stage kt + 3's scales into slot q, stage kt + 1's activations into A buffer r ^ 1,
  // stage kt + 3's weight chunk into slot q; then stage kt + 1's widened weights (slot
  // q + 1, loaded in stage kt - 2) into B buffer r ^ 1; multiply buffer r; wait for
  // stage kt + 1's activations: exactly one load (the weight chunk) was issued after
  // them and vector loads complete in order, so vmcnt(1) covers them while the weight
  // chunk stays in flight.
  auto stage = [&](auto rc, auto qc, int kt) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::v, q = decltype(qc)::v;
    const int k0 = kt * BK;
    __builtin_amdgcn_sched_barrier(0);
    load_s(k0 + 3 * BK, sreg0(qc), sreg1(qc));
    __builtin_amdgcn_sched_barrier(0);
    dma_a(abuf(Ring<r ^ 1>{}), k0 + BK);  // past the end: zeros / unused
    __builtin_amdgcn_sched_barrier(0);
    load_w(k0 + 3 * BK, wreg(qc));
    __builtin_amdgcn_sched_barrier(0);
    store_b(Ring<r ^ 1>{}, wreg(Ring<(q + 1) % 3>{}), sreg0(Ring<(q + 1) % 3>{}), sreg1(Ring<(q + 1) % 3>{}));
    const uint4* as = abuf(rc);
    const uint4* bs = bbuf(rc);
    auto kstep = [&](auto ksc) __attribute__((always_inline)) {
      constexpr int ks = decltype(ksc)::v;
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
      // Every subtile is multiplied, those past the segment on zero rows: a branch per
      // subtile would cut the stage into basic blocks that the widening and the LDS
      // traffic cannot be scheduled across (measured: config E 224 -> 210 us).
#pragma unroll
      for (int j = 0; j < TMX; ++j) {
#pragma unroll
        for (int i = 0; i < TN; ++i) accg[i][j] = Mfma16<MT>::mma(bop[i], aop[j], accg[i][j]);
      }
      if ((k0 + 32 * (ks + 1)) % p.group == 0) {  // group ends
        // the scales of this lane's 4 TN columns, read only here (the 1/16 of the
        // widening is applied once, in the epilogue)
        float sc[TN][4];
        if constexpr (STAB) {
          // accg is never cleared: it holds T_g = P_0 + ... + P_g, the products of all
          // groups so far, and sum_g s_g P_g = sum_g (s_g - s_{g+1}) T_g with s_G = 0
          // (summation by parts), one FMA per accumulator and group instead of an FMA
          // and a clear
          const int g = (k0 + 32 * ks) / p.group;
          const int gn = min(g + 1, G_blk - 1);
          const float keep = g + 1 < G_blk ? 1.f : 0.f;
#pragma unroll
          for (int i = 0; i < TN; ++i) {
            const uint2 h2 = *reinterpret_cast<const uint2*>(sT + g * BN + wn * 64 + i * 16 + 4 * lk);
            const uint2 n2 = *reinterpret_cast<const uint2*>(sT + gn * BN + wn * 64 + i * 16 + 4 * lk);
            const _Float16* h = reinterpret_cast<const _Float16*>(&h2);
            const _Float16* hn = reinterpret_cast<const _Float16*>(&n2);
#pragma unroll
            for (int q = 0; q < 4; ++q) sc[i][q] = fmaf(-keep, (float)hn[q], (float)h[q]);
          }
#pragma unroll
          for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TMX; ++j)
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[i][j][q] = fmaf(sc[i][q], accg[i][j][q], acc[i][j][q]);
        } else {
#pragma unroll
          for (int i = 0; i < TN; ++i) {
            const float4 s4 = *reinterpret_cast<const float4*>(sS + (r * 2 + ks) * BN + wn * 64 + i * 16 + 4 * lk);
            sc[i][0] = s4.x;
            sc[i][1] = s4.y;
            sc[i][2] = s4.z;
            sc[i][3] = s4.w;
          }
          // acc += s[n] * partial, and a fresh partial for the next group
#pragma unroll
          for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TMX; ++j) {
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[i][j][q] = fmaf(sc[i][q], accg[i][j][q], acc[i][j][q]);
              accg[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
      }
    };
    kstep(Ring<0>{});
    kstep(Ring<1>{});
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue: stage 0 into buffers 0; stages 1 and 2's weights into slots 1 and 2
  dma_a(As0, 0);
  load_w(0, w0);
  load_s(0, s00, s01);
  __builtin_amdgcn_s_waitcnt(0);
  store_b(Ring<0>{}, w0, s00, s01);
  load_w(BK, w1);
  load_s(BK, s10, s11);
  load_w(2 * BK, w2);
  load_s(2 * BK, s20, s21);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // six stages per trip (LDS buffer kt % 2, register slot kt % 3), leaving after any
  if (nk > 0) {
    for (int kt = 0;; kt += 6) {
      stage(Ring<0>{}, Ring<0>{}, kt);
      if (kt + 1 >= nk) break;
      stage(Ring<1>{}, Ring<1>{}, kt + 1);
      if (kt + 2 >= nk) break;
      stage(Ring<0>{}, Ring<2>{}, kt + 2);
      if (kt + 3 >= nk) break;
      stage(Ring<1>{}, Ring<0>{}, kt + 3);
      if (kt + 4 >= nk) break;
      stage(Ring<0>{}, Ring<1>{}, kt + 4);
      if (kt + 5 >= nk) break;
      stage(Ring<1>{}, Ring<2>{}, kt + 5);
      if (kt + 6 >= nk) break;
    }
  }
  // loads past the end may still be in flight: drain them before the LDS is reused
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: acc[i][j][r] = C[m = m0 + (2 j + wm) 16 + lr][n = n0 + 64 wn + 16 i + 4 lk + r]
  OT* c = static_cast<OT*>(p.c) + (int64_t)split * p.c_sstride;
  if constexpr (GU) {
    // wavefronts wn = 1 hold the up products: they pass them through LDS (the
    // activation buffers, free now) to the wavefronts wn = 0, which hold the gate
    // products of the same (m, n) and write silu(gate) * up. Subtile q = 2 j + wm
    // (16 rows x 64 columns fp32, 4 KiB) goes to buffer q % 2 at 4 KiB (q / 2): the
    // TMX subtiles of one parity fill one TMX x 4 KiB buffer exactly.
    // Inside a subtile, row lr's 16-byte column chunk 4 i + lk sits at chunk (4 i + lk) ^
    // (lr & 7): rows are 256 bytes apart, so without the XOR the 8 rows of one access
    // would share their banks.
    auto ubuf = [&](int q) __attribute__((always_inline)) -> float* {
      uint4* b = (q & 1) ? As1 : As0;
      return reinterpret_cast<float*>(b) + (q >> 1) * 1024;
    };
    auto uoff = [&](int i) __attribute__((always_inline)) { return lr * 64 + (((4 * i + lk) ^ (lr & 7)) * 4); };
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TMX; ++j) *reinterpret_cast<f32x4*>(ubuf(2 * j + wm) + uoff(i)) = acc[i][j];
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
        const f32x4 u = *reinterpret_cast<const f32x4*>(ubuf(2 * j + wm) + uoff(i));
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float g = acc[i][j][r] * 0.0625f;
          v[r] = g / (1.0f + __expf(-g)) * (u[r] * 0.0625f);
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
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc[i][j][r] * 0.0625f;  // the widening's 16 (v - 8)
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

template <typename MT, int TMX, int SCL, bool GU, typename OT = MT>
static int launch_grouped(Mfma16Params p, hipStream_t st) {
  constexpr int BMX = 32 * TMX, OUTN = GU ? 64 : 128;
  p.n_tiles = (int)cdiv(p.N, OUTN);
  // upper bound on sum_e ceil(rows_e / BMX) without reading the device offsets
  p.m_tiles = (int)(cdiv(p.M, BMX) + p.E);
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles * (p.ksplit > 1 ? p.ksplit : 1);
  if (blocks > 0x7FFFFFFF) return MLS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((grouped_int4_kernel<MT, OT, TMX, SCL, GU>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  return check_launch(GU ? "grouped INT4 gate/up GEMM" : "grouped INT4 GEMM");
}

template <int SCL, bool GU>
static int launch_grouped_tmx(const Mfma16Params& p, hipStream_t st, bool bf16, int tmx) {
  switch (tmx) {
    case 5:
      if constexpr (SCL >= 32)
        return bf16 ? launch_grouped<__bf16, 5, SCL, GU>(p, st) : launch_grouped<_Float16, 5, SCL, GU>(p, st);
      [[fallthrough]];  // per-stage scales: 160-row chunks are not built (they would spill)
    case 4: return bf16 ? launch_grouped<__bf16, 4, SCL, GU>(p, st) : launch_grouped<_Float16, 4, SCL, GU>(p, st);
    case 3: return bf16 ? launch_grouped<__bf16, 3, SCL, GU>(p, st) : launch_grouped<_Float16, 3, SCL, GU>(p, st);
    default: return bf16 ? launch_grouped<__bf16, 2, SCL, GU>(p, st) : launch_grouped<_Float16, 2, SCL, GU>(p, st);
  }
}

// Row-chunk height: the smallest of 64 / 96 / 128 / 160 rows that holds 1.25x the
// average segment (routed segments scatter around the average), so a typical expert's
// rows fit in one chunk and its weights are streamed and widened once.
// MLS_GROUPED_TMX (2..5) overrides the chunk height (32 TMX rows) for sweeps.
static int chunk_tmx(int64_t M, int E) {
  const int64_t want = cdiv(M * 5, (int64_t)E * 4);
  static const int tmx_env = env_int("MLS_GROUPED_TMX", 0);
  return tmx_env >= 2 && tmx_env <= 5 ? tmx_env : want > 128 ? 5 : want > 96 ? 4 : want > 64 ? 3 : 2;
}

int grouped_splits(int64_t M, int E, int64_t N, int64_t K, int group) {
  // MLS_GROUPED_SPLITS (1, 2, 4, 8) forces the split count for sweeps
  static const int env = env_int("MLS_GROUPED_SPLITS", 0);
  if (M <= 0 || E <= 0 || N <= 0 || K <= 0 || group <= 0) return 1;
  const int64_t tiles = cdiv(N, 128) * (cdiv(M, 32 * chunk_tmx(M, E)) + E / 2);
  int best = 1;
  for (int s = 1; s <= 8; s *= 2) {
    const int64_t kp = K / s;
    // each range: a multiple of 64 and of the group, its scales in the 32-group table
    const bool ok = K % s == 0 && kp % 64 == 0 && kp % group == 0 && kp / group <= 32 && (kp / group) % 4 == 0;
    if (env > 0) {
      if (s == env) return ok ? s : 1;
      continue;
    }
    if (ok) {
      best = s;
      if (tiles * s >= 512) break;  // two blocks per CU reached
    }
  }
  return env > 0 ? 1 : best;
}

template <int SCL>
static int launch_partial_tmx(const Mfma16Params& p, hipStream_t st, bool bf16, int tmx) {
  switch (tmx) {
    case 5:
      if constexpr (SCL >= 32)
        return bf16 ? launch_grouped<__bf16, 5, SCL, false, float>(p, st)
                    : launch_grouped<_Float16, 5, SCL, false, float>(p, st);
      [[fallthrough]];  // per-stage scales: 160-row chunks are not built (they would spill)
    case 4: return bf16 ? launch_grouped<__bf16, 4, SCL, false, float>(p, st) : launch_grouped<_Float16, 4, SCL, false, float>(p, st);
    case 3: return bf16 ? launch_grouped<__bf16, 3, SCL, false, float>(p, st) : launch_grouped<_Float16, 3, SCL, false, float>(p, st);
    default: return bf16 ? launch_grouped<__bf16, 2, SCL, false, float>(p, st) : launch_grouped<_Float16, 2, SCL, false, float>(p, st);
  }
}

int launch_grouped_partial(const Mfma16Params& p, hipStream_t st, bool bf16) {
  const int s = p.ksplit;
  if (s < 1 || p.K % s != 0) return MLS_ERR_UNSUPPORTED;
  const int64_t kp = p.K / s, G = kp / p.group;
  if (kp % 64 != 0 || kp % p.group != 0) return MLS_ERR_UNSUPPORTED;
  const int tmx = chunk_tmx(p.M, p.E);
  const bool stab = p.s_dt == MLS_F16 && p.ld_sg == 1 && G % 4 == 0 && G <= 32 && (p.ld_sn % 4) == 0 &&
                    (p.s_estride % 4) == 0 && aligned(p.s, 8);
  if (stab) return launch_partial_tmx<32>(p, st, bf16, tmx);
  if (p.s_dt == MLS_F16) return launch_partial_tmx<1>(p, st, bf16, tmx);
  return launch_partial_tmx<0>(p, st, bf16, tmx);
}

int launch_grouped_seg(const Mfma16Params& p, hipStream_t st, bool bf16, bool gate_up) {
  const int tmx = chunk_tmx(p.M, p.E);
  // scale table in LDS: fp16 scales, contiguous groups, G a multiple of 4 up to 128,
  // 8-byte aligned rows; a table of up to 32 groups keeps two blocks per CU
  const int64_t G = p.K / p.group;
  const bool stab = p.s_dt == MLS_F16 && p.ld_sg == 1 && G % 4 == 0 && G <= 128 && (p.ld_sn % 4) == 0 &&
                    (p.s_estride % 4) == 0 && aligned(p.s, 8) && (!gate_up || aligned(p.s2, 8));
  if (!stab && p.s_dt == MLS_F16)
    return gate_up ? launch_grouped_tmx<1, true>(p, st, bf16, tmx) : launch_grouped_tmx<1, false>(p, st, bf16, tmx);
  if (!stab)
    return gate_up ? launch_grouped_tmx<0, true>(p, st, bf16, tmx) : launch_grouped_tmx<0, false>(p, st, bf16, tmx);
  if (G <= 32)
    return gate_up ? launch_grouped_tmx<32, true>(p, st, bf16, tmx) : launch_grouped_tmx<32, false>(p, st, bf16, tmx);
  return gate_up ? launch_grouped_tmx<128, true>(p, st, bf16, tmx) : launch_grouped_tmx<128, false>(p, st, bf16, tmx);
}

}  // namespace mls
