// Large GEMMs on the 16-bit MFMA (v_mfma_f32_16x16x32_{bf16,f16}) whose byte-wide operands
// stay bytes until they leave LDS: the exact e4m3 / e5m2 GEMM (both fp8 operands widened to
// bf16, exact). The kernel also takes 16-bit A with INT8 B (weight-only prefill, row scale
// per n), which measured slower than the register-staged kernel (gemm_mfma16.hip) and is
// not dispatched: widening each byte per wavefront instead of once per block raises the
// VALU per MFMA from 2.2 to 2.9.
//
// Block tile BM (rows m of A) x BN (rows n of B) x 64 (k), 8 wavefronts (two per SIMD) as
// WM x WN, each with a (BM / WM) x (BN / WN) output tile. Every operand enters LDS through
// buffer loads that write LDS directly (buffer_load_dwordx4 ... lds): no staging registers,
// no ds_write, and INT8 / fp8 tiles cost half the LDS of their 16-bit widening. A wavefront
// reads each 16-byte byte chunk once per stage and widens it in registers (INT8: exact
// integers, 6 VALU per 4 weights; e4m3 / e5m2: v_cvt_scalef32_pk_bf16_fp8 / _bf8 with scale
// 1, exact) right before its MFMAs.
//
// Three LDS buffers per operand (two stages of loads in flight); per stage, one barrier:
//   1. issue the LDS-direct loads of stage s + 2 into the buffer stage s - 1 used,
//   2. read stage s's operands from LDS, widen and multiply,
//   3. wait for this wavefront's loads of stage s + 1 (vmcnt) and barrier.
// The compiler holds an LDS read behind every pending LDS-direct load it cannot prove
// disjoint from it, which would serialise each stage behind the prefetch just issued; the
// operand reads are therefore inline-asm ds_read_b128, each use tied to an explicit
// lgkmcnt wait (LDS reads complete in order, and no scalar-memory load is in flight
// inside the loop), and the buffers rotate without the compiler tracking them.
//
// k order inside a stage: MFMA k-slot (ks, g) of lane group g = lane / 16 holds the 8
// values k = 16 g + 8 ks + [0, 8), so one 16-byte byte chunk (k = 16 g .. 16 g + 15) feeds
// both MFMA k-steps; a 16-bit operand reads its two 16-byte chunks 2 g + ks. Both operands
// use the same order, and the MFMA sums over all of them.
//
// LDS rows: 16-bit rows are 128 bytes, byte rows 64 bytes, with the 16-byte chunks
// permuted per row (RowFmt) so that the 16 rows of an operand read spread over all banks.
//
// The B tile is the MFMA "A" operand, so lane l's accumulator holds C[n = 4 (l / 16) + i]
// [m = l % 16], i = 0..3: 4 consecutive outputs of one row m per store.
#include <utility>

#include "mfma16.h"

namespace mls {

namespace {

constexpr int kWaves = 8;

// Where logical 16-byte chunk lc of a row sits in LDS, and back. Byte rows: lc ^ ((row >>
// 1) & 3). 16-bit rows: the chunk index is first rotated, pi(c) = 4 (c & 1) + (c >> 1),
// then XOR-ed with row & 7: the MFMA step ks of lane group g reads chunk 2 g + ks, which
// lands at (4 ks + g) ^ (row & 7), the placement that measured free of bank conflicts
// for 16-row operand reads (the unrotated 2 g + ks measured 3.4 conflict cycles per read).
template <bool BYTES>
struct RowFmt {
  static constexpr int BYTES_PER_ROW = BYTES ? 64 : 128;
  static constexpr int CHUNKS = BYTES_PER_ROW / 16;
  __device__ static __forceinline__ int phys(int row, int lc) {
    return BYTES ? (lc ^ ((row >> 1) & 3)) : ((((lc & 1) << 2) | (lc >> 1)) ^ (row & 7));
  }
  __device__ static __forceinline__ int logical(int row, int pc) {
    if (BYTES) return pc ^ ((row >> 1) & 3);
    const int q = pc ^ (row & 7);
    return ((q & 3) << 1) | (q >> 2);
  }
};

// LDS-direct fill of one operand stage: ROWS rows of RowFmt<BYTES>, 16-byte slots spread
// over the block's wavefronts by whole instructions (instruction i of the tile belongs to
// wavefront i % 8). Slot s of the tile: row s / CHUNKS, physical chunk s % CHUNKS, which
// holds logical chunk RowFmt::logical(row, s % CHUNKS).
template <int ROWS, bool BYTES>
struct Filler {
  using F = RowFmt<BYTES>;
  static constexpr int INSTR = ROWS * F::CHUNKS / 64;  // 64 slots per instruction
  static constexpr int PER_WAVE = (INSTR + kWaves - 1) / kWaves;
  static_assert(ROWS * F::CHUNKS % 64 == 0, "whole instructions");
  int off[PER_WAVE];
  __device__ __forceinline__ void init(int wave, int lane, int ld_bytes) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int s = (i * kWaves + wave) * 64 + lane;
      const int row = s / F::CHUNKS, pc = s % F::CHUNKS;
      off[i] = row * ld_bytes + F::logical(row, pc) * 16;
    }
  }
  // instructions wavefront `wave` issues per stage
  __device__ static __forceinline__ int count(int wave) {
    return INSTR / kWaves + (wave < INSTR % kWaves ? 1 : 0);
  }
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int wave, int k_bytes) const {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i)
      if (INSTR % kWaves == 0 || i * kWaves + wave < INSTR)
        lds_load16(rs, lds + (i * kWaves + wave) * 1024, off[i], k_bytes);
  }
};

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 8] (the count is an immediate)
__device__ __forceinline__ void wait_vmcnt_upto8(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0 | 0x70 | 0xF00); break;
    case 1: __builtin_amdgcn_s_waitcnt(1 | 0x70 | 0xF00); break;
    case 2: __builtin_amdgcn_s_waitcnt(2 | 0x70 | 0xF00); break;
    case 3: __builtin_amdgcn_s_waitcnt(3 | 0x70 | 0xF00); break;
    case 4: __builtin_amdgcn_s_waitcnt(4 | 0x70 | 0xF00); break;
    case 5: __builtin_amdgcn_s_waitcnt(5 | 0x70 | 0xF00); break;
    case 6: __builtin_amdgcn_s_waitcnt(6 | 0x70 | 0xF00); break;
    case 7: __builtin_amdgcn_s_waitcnt(7 | 0x70 | 0xF00); break;
    default: __builtin_amdgcn_s_waitcnt(8 | 0x70 | 0xF00); break;
  }
}

// Block-wide meeting point after this wavefront's LDS-direct loads but the last n have
// landed. s_barrier alone orders nothing for the compiler: the empty asm statements with a
// memory clobber keep every LDS access on its side of the barrier (a __syncthreads()
// would do that too, but its fence waits for every load in flight, vmcnt(0)).
__device__ __forceinline__ void block_sync(int n) {
  asm volatile("" ::: "memory");
  wait_vmcnt_upto8(n);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 to_uint4(u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

// LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte LDS read issued as inline asm: its value is valid only after an lgkmcnt wait
// tied to it (lgkm_wait1 / lgkm_wait_tied), which the caller places.
template <int OFF>
__device__ __forceinline__ u32x4 ds_read16(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset");
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// s_waitcnt lgkmcnt(N) that the uses of v must follow
template <int N>
__device__ __forceinline__ void lgkm_wait1(u32x4& v) {
  static_assert(N >= 0 && N < 16, "lgkmcnt");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(N));
}

// s_waitcnt lgkmcnt(N) that the uses of every element of a[TM][AKS] must follow
template <int N, int TM, int AKS>
__device__ __forceinline__ void lgkm_wait_tied(u32x4 (&a)[TM][AKS]) {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N));
#pragma unroll
  for (int j = 0; j < TM; ++j)
#pragma unroll
    for (int h = 0; h < AKS; ++h) asm volatile("" : "+v"(a[j][h]));
}

template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

template <int AKIND, int BKIND, typename MT, typename OT, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * kWaves) void gemm_bytes_kernel(const Mfma16Params p) {
  static_assert(WM * WN == kWaves, "8 wavefronts");
  constexpr bool A8 = AKIND != A_RAW16;
  static_assert(BKIND == B_INT8 || BKIND == B_E4M3, "byte-wide B");
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 16, TN = WTN / 16;
  // PRIO: a wavefront raises its issue priority (s_setprio 1) while it widens and multiplies
  // and drops it before the barrier, so the other wavefront of its SIMD issues its LDS reads
  // in the gaps. Measured on one box: exact e4m3 at config D -1.7% (three A/B pairs); the
  // e5m2 x e4m3 backward GEMMs +0.5%, so only the e4m3 x e4m3 kernel does it.
  constexpr bool PRIO = AKIND == A_E4M3;
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "16-row MFMA tiles");
  using FA = Filler<BM, A8>;
  using FB = Filler<BN, true>;
  constexpr int A_STAGE = BM * RowFmt<A8>::BYTES_PER_ROW, B_STAGE = BN * 64;

  extern __shared__ __align__(16) uint8_t smem[];  // A [3][A_STAGE], then B [3][B_STAGE]
  const uint32_t lds0 = lds_addr(smem);

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  int nt, mt;
  tile_order(L, p.m_tiles, p.n_tiles, p.tile_gm, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int M = p.M, N = p.N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
  const int lr = lane & 15, g = lane >> 4;

  constexpr int AES = A8 ? 1 : 2;  // bytes per A element
  const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.a + (int64_t)m0 * p.lda * AES), (short)0, (int)(rows_a * p.lda * AES), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.b + (int64_t)n0 * p.ldb), (short)0, (int)(rows_b * p.ldb), 0x00020000);
  FA fa;
  FB fb;
  fa.init(wave, lane, (int)p.lda * AES);
  fb.init(wave, lane, (int)p.ldb);
  // LDS-direct loads this wavefront issues per stage (the tiles' instructions are dealt
  // out round-robin, so the first INSTR % 8 wavefronts may carry one more)
  const int per_stage = FA::count(wave) + FB::count(wave);

  // This lane's operand chunks inside a stage, as a base address plus per-tile immediate
  // offsets: rows wm0 + 16 j + lr share (row & 7) = (lr & 7) and ((row >> 1) & 3) =
  // ((lr >> 1) & 3), so the swizzled chunk depends on the lane only.
  constexpr int AKS = A8 ? 1 : 2;  // A reads per tile and stage
  uint32_t a_base[AKS];
#pragma unroll
  for (int h = 0; h < AKS; ++h) {
    const int row = wm0 + lr;
    a_base[h] = A8 ? (uint32_t)(row * 64 + RowFmt<true>::phys(row, g) * 16)
                   : (uint32_t)(row * 128 + RowFmt<false>::phys(row, 2 * g + h) * 16);
  }
  const uint32_t b_base = 3 * A_STAGE + (uint32_t)((wn0 + lr) * 64 + RowFmt<true>::phys(wn0 + lr, g) * 16);
  constexpr int A_TSTRIDE = 16 * RowFmt<A8>::BYTES_PER_ROW, B_TSTRIDE = 16 * 64;

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / 64;
  fa.issue(rsa, smem, wave, 0);
  fb.issue(rsb, smem + 3 * A_STAGE, wave, 0);
  if (nk > 1) {
    fa.issue(rsa, smem + A_STAGE, wave, 64 * AES);
    fb.issue(rsb, smem + 3 * A_STAGE + B_STAGE, wave, 64);
  }
  block_sync(nk > 1 ? per_stage : 0);

  int cur = 0;  // buffer of stage kt: kt % 3
  for (int kt = 0; kt < nk; ++kt) {
    const int nxt2 = cur == 0 ? 2 : cur - 1;  // (kt + 2) % 3
    __builtin_amdgcn_sched_barrier(0);
    // 1. stage kt + 2 into the buffer stage kt - 1 used
    const bool more = kt + 2 < nk;
    if (more) {
      fa.issue(rsa, smem + nxt2 * A_STAGE, wave, (kt + 2) * 64 * AES);
      fb.issue(rsb, smem + 3 * A_STAGE + nxt2 * B_STAGE, wave, (kt + 2) * 64);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2. this stage's operands (asm reads: the compiler would otherwise wait for the
    // LDS-direct loads just issued before every LDS read)
    const uint32_t sa = lds0 + cur * A_STAGE, sb = lds0 + cur * B_STAGE;
    u32x4 araw[TM][AKS], braw[TN];
    static_for<TM>([&](auto J) {
      static_for<AKS>([&](auto H) {
        araw[J.value][H.value] = ds_read16<J.value * A_TSTRIDE>(sa + a_base[H.value]);
      });
    });
    static_for<TN>([&](auto I) { braw[I.value] = ds_read16<I.value * B_TSTRIDE>(sb + b_base); });
    // 3. widen and multiply as the reads land (LDS reads complete in order)
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
    lgkm_wait_tied<TN>(araw);
    uint4 aop[TM][2];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      if constexpr (A8) {
        uint32_t o[8];
        const uint4 raw = to_uint4(araw[j][0]);
        if constexpr (AKIND == A_E5M2)
          widen_e5m2(raw, o);
        else
          widen_e4m3(raw, o);
        aop[j][0] = make_uint4(o[0], o[1], o[2], o[3]);
        aop[j][1] = make_uint4(o[4], o[5], o[6], o[7]);
      } else {
        aop[j][0] = to_uint4(araw[j][0]);
        aop[j][1] = to_uint4(araw[j][1]);
      }
    }
    static_for<TN>([&](auto I) {
      constexpr int i = I.value;
      lgkm_wait1<TN - 1 - i>(braw[i]);
      uint32_t o[8];
      if constexpr (BKIND == B_INT8)
        widen_int8<MT>(to_uint4(braw[i]), o);
      else
        widen_e4m3(to_uint4(braw[i]), o);
      const uint4 b0 = make_uint4(o[0], o[1], o[2], o[3]), b1 = make_uint4(o[4], o[5], o[6], o[7]);
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        acc[i][j] = Mfma16<MT>::mma(b0, aop[j][0], acc[i][j]);
        acc[i][j] = Mfma16<MT>::mma(b1, aop[j][1], acc[i][j]);
      }
    });
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
    // 4. this wavefront's loads of stage kt + 1 have landed; after the barrier everyone's
    // have, and nobody reads this stage's buffer again before it is refilled
    block_sync(more ? per_stage : 0);
    cur = cur == 2 ? 0 : cur + 1;
  }

  // ---- epilogue: acc[i][j][r] = C[m = m0+wm0+16j+lr][n = n0+wn0+16i+4g+r]
  OT* c = static_cast<OT*>(p.c);
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn0 + i * 16 + 4 * g;
    float sn[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = min(nb + r, N - 1);
      if constexpr (BKIND == B_INT8)
        sn[r] = scale_at(p.s, p.s_dt, n * p.ld_sn);
      else
        sn[r] = p.sbp ? p.sbp[(int64_t)n * p.sbs] : p.sb;
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int m = m0 + wm0 + j * 16 + lr;
      if (m >= M) continue;
      float sm = 1.f;
      if constexpr (BKIND == B_E4M3) sm = p.sap ? p.sap[(int64_t)m * p.sas] : p.sa;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = BKIND == B_E4M3 ? acc[i][j][r] * (sm * sn[r]) : acc[i][j][r] * sn[r];
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

template <int AKIND, int BKIND, typename MT, typename OT, int BM, int BN, int WM, int WN>
int launch_bytes(Mfma16Params p, hipStream_t st) {
  p.n_tiles = (int)cdiv(p.N, BN);
  p.m_tiles = (int)cdiv(p.M, BM);
  static const int gm = env_int("MLS_TILE_GM", 4);  // row tiles per run of the tile order (0: column-major)
  p.tile_gm = gm;
  constexpr size_t lds = (size_t)3 * (BM * RowFmt<AKIND != A_RAW16>::BYTES_PER_ROW + BN * 64);
  auto kern = gemm_bytes_kernel<AKIND, BKIND, MT, OT, BM, BN, WM, WN>;
  static bool attr_set = false;  // raise the dynamic LDS limit once per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
        hipSuccess)
      return fail(MLS_ERR_HIP, "byte-operand GEMM: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  const int64_t blocks = (int64_t)p.n_tiles * p.m_tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * kWaves), lds, st, p);
  return check_launch("byte-operand GEMM");
}

// Tuning override for sweeps: MLS_BYTES_SHAPE = BN * 10 + layout (layout 0: 4 x 2
// wavefronts of 64 x (BN / 2); 1: 2 x 4 of 128 x (BN / 4)); BM is 256.
template <int AKIND, int BKIND, typename MT, typename OT>
int dispatch_bytes(const Mfma16Params& p, hipStream_t st) {
  static const int force = env_int("MLS_BYTES_SHAPE", 0);
  int bn = 256, layout = 0;
  if (force) {
    bn = force / 10;
    layout = force % 10;
  } else {
    // 256 x 192 tiles when fewer rounds of 256 blocks outweigh the smaller tile (2048 x
    // 11008: 344 blocks of 256 x 256 are 1.34 rounds, 464 of 256 x 192 are 1.81)
    const int64_t mt = cdiv(p.M, 256);
    const int64_t c256 = cdiv(mt * cdiv(p.N, 256), 256) * 256, c192 = cdiv(mt * cdiv(p.N, 192), 256) * 192;
    if (c192 < c256) bn = 192;
  }
  if (bn == 192) {
    return layout ? launch_bytes<AKIND, BKIND, MT, OT, 256, 192, 4, 2>(p, st)  // 64 x 96
                  : launch_bytes<AKIND, BKIND, MT, OT, 256, 192, 2, 4>(p, st);  // 128 x 48
  }
  return layout ? launch_bytes<AKIND, BKIND, MT, OT, 256, 256, 2, 4>(p, st)  // 128 x 64
                : launch_bytes<AKIND, BKIND, MT, OT, 256, 256, 4, 2>(p, st);  // 64 x 128
}

}  // namespace

int launch_bytes_fp8(const Mfma16Params& p, hipStream_t st, bool a_e5m2, int c_dt) {
  if (a_e5m2) {
    if (c_dt == MLS_F32) return dispatch_bytes<A_E5M2, B_E4M3, __bf16, float>(p, st);
    if (c_dt == MLS_F16) return dispatch_bytes<A_E5M2, B_E4M3, __bf16, _Float16>(p, st);
    return dispatch_bytes<A_E5M2, B_E4M3, __bf16, __bf16>(p, st);
  }
  if (c_dt == MLS_F32) return dispatch_bytes<A_E4M3, B_E4M3, __bf16, float>(p, st);
  if (c_dt == MLS_F16) return dispatch_bytes<A_E4M3, B_E4M3, __bf16, _Float16>(p, st);
  return dispatch_bytes<A_E4M3, B_E4M3, __bf16, __bf16>(p, st);
}

}  // namespace mls
