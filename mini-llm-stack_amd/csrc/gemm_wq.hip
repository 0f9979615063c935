// Prefill-shaped weight-only GEMM on bf16/fp16 MFMA (v_mfma_f32_16x16x32_{bf16,f16}).
//
// Block tile BM (activation rows m) x BN (weight rows n) x 64 (k), 256 threads as
// WM x WN wavefronts. Per k-stage every thread
//   - prefetches its share of the next stage (16-byte loads of activations and
//     of packed weights, plus INT4 group scales) into registers,
//   - runs the MFMAs of the current stage out of LDS,
//   - dequantizes its prefetched weights to 16-bit floats in registers (INT8:
//     exact integers, scale applied in the epilogue; INT4: (v - 8) * s rounded
//     once, like the reference kernel's w.to(a.dtype)) and stores both tiles into
//     the other LDS buffer,
// with one barrier per stage. LDS rows are 64 k = 128 bytes, and the 16-byte
// chunk index is XOR-swizzled with (row & 7) so the 16 lanes that read one MFMA
// operand column hit distinct banks.
//
// The MFMA is issued with the weight tile as the "A" operand, so each lane's
// accumulator holds 4 consecutive n of one m: the epilogue multiplies 4
// consecutive scales and writes 4 consecutive outputs with one store.
//
// GROUPED = true runs the per-expert variant for MoE: rows of `a` are sorted by
// expert, seg_off (device) gives each expert's row range, and each block
// resolves (expert, m-tile) from seg_off on the device.
#include "wq.h"

namespace mls {

template <typename AT> struct Mfma16;
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

__device__ __forceinline__ float scale_at(const void* s, int s_dt, int64_t i) {
  return s_dt == MLS_F16 ? (float)((const _Float16*)s)[i] : ((const float*)s)[i];
}

__device__ __forceinline__ float u8f(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }

// 16 INT8 weights (one 16-byte chunk) -> 16 exact 16-bit floats (8 dwords).
template <typename AT>
__device__ __forceinline__ void deq_int8(const uint4& q, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t u = d[t] ^ 0x80808080u;  // q + 128
    o[2 * t + 0] = Mfma16<AT>::pack2(u8f(u, 0) - 128.0f, u8f(u, 1) - 128.0f);
    o[2 * t + 1] = Mfma16<AT>::pack2(u8f(u, 2) - 128.0f, u8f(u, 3) - 128.0f);
  }
}

// 32 INT4 weights (one 16-byte chunk, one scale group) -> 32 16-bit floats (16 dwords),
// w = (v - 8) * s rounded once.
template <typename AT>
__device__ __forceinline__ void deq_int4(const uint4& q, float s, uint32_t* o) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
  const float m8s = -8.0f * s;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = d[t] & 0x0F0F0F0Fu;         // k = 8t + 0, 2, 4, 6
    const uint32_t hi = (d[t] >> 4) & 0x0F0F0F0Fu;  // k = 8t + 1, 3, 5, 7
#pragma unroll
    for (int b = 0; b < 4; ++b)
      o[4 * t + b] = Mfma16<AT>::pack2(fmaf(u8f(lo, b), s, m8s), fmaf(u8f(hi, b), s, m8s));
  }
}

template <int WBITS, typename AT, int BM, int BN, int WM, int WN, bool GROUPED>
__global__ __launch_bounds__(256) void gemm_wq_mfma_kernel(
    const AT* __restrict__ a, int64_t lda, const uint8_t* __restrict__ w, int64_t ldw,
    const void* __restrict__ s, int s_dt, int64_t ld_sn, int64_t ld_sg, int group,
    AT* __restrict__ c, int64_t ldc, int M, int N, int K, int n_tiles, int m_tiles,
    const int32_t* __restrict__ seg_off, int E, int64_t w_estride, int64_t s_estride) {
  constexpr int BK = 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 16, TN = WTN / 16;  // MFMA tiles per wave
  static_assert(WM * WN == 4 && TM >= 1 && TN >= 1, "bad wave layout");
  constexpr int A_CH = BM * 8;                  // 16-byte chunks of the A stage
  constexpr int A_PT = (A_CH + 255) / 256;      // per thread
  constexpr int WCPR = WBITS == 8 ? 4 : 2;      // 16-byte weight chunks per row per stage
  constexpr int B_CH = BN * WCPR;
  static_assert(B_CH % 256 == 0, "BN too small");
  constexpr int B_PT = B_CH / 256;
  constexpr int KPC = WBITS == 8 ? 16 : 32;     // k per weight chunk

  extern __shared__ __align__(16) uint8_t smem[];
  uint4* As = reinterpret_cast<uint4*>(smem);                // [2][BM][8] chunks
  uint4* Bs = As + 2 * BM * 8;                                // [2][BN][8] chunks

  // ---- which tile
  const int nblocks = gridDim.x;
  const int L = xcd_remap(blockIdx.x, nblocks);
  const int nt = L / m_tiles, mt = L % m_tiles;  // consecutive L share a weight tile
  if (nt >= n_tiles) return;
  int row_lo = 0, row_hi = M, m0;
  if constexpr (GROUPED) {
    int e = 0, cum = 0;
    for (; e < E; ++e) {
      const int lo = seg_off[e], hi = seg_off[e + 1];
      const int t = (hi - lo + BM - 1) / BM;
      if (mt < cum + t) {
        row_lo = lo;
        row_hi = hi;
        break;
      }
      cum += t;
    }
    if (e == E) return;  // surplus block
    m0 = row_lo + (mt - cum) * BM;
    w += (int64_t)e * w_estride;
    s = (const uint8_t*)s + (int64_t)e * s_estride * (s_dt == MLS_F16 ? 2 : 4);
  } else {
    m0 = mt * BM;
  }
  const int n0 = nt * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;

  // ---- per-thread staging: buffer descriptors cover only this tile's valid rows
  // (rows past the segment / N read as zeros); the stage offset is the scalar offset.
  constexpr int ESZ = sizeof(AT);
  const int rows_a = min(BM, row_hi - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a + (int64_t)m0 * lda), (short)0, (int)(rows_a * lda * ESZ), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (int64_t)n0 * ldw), (short)0, (int)(rows_b * ldw), 0x00020000);
  // A chunk q = tid + 256 i: row (tid >> 3) + 32 i, 16-byte chunk tid & 7
  const int a_row0 = tid >> 3, a_kc = tid & 7;
  const int a_lds0 = a_row0 * 8 + (a_kc ^ (a_row0 & 7));
  int a_off[A_PT];
#pragma unroll
  for (int i = 0; i < A_PT; ++i) a_off[i] = (a_row0 + 32 * i) * (int)lda * ESZ + a_kc * 16;
  // weight chunk q = tid + 256 i: row q / WCPR, chunk q % WCPR
  constexpr int RSTEP = 256 / WCPR;
  const int b_row0 = tid / WCPR, b_cc = tid % WCPR;
  int b_off[B_PT];
  int64_t b_srow[B_PT];
#pragma unroll
  for (int i = 0; i < B_PT; ++i) {
    b_off[i] = (b_row0 + RSTEP * i) * (int)ldw + b_cc * 16;
    b_srow[i] = (int64_t)min(n0 + b_row0 + RSTEP * i, N - 1) * ld_sn;
  }
  const bool a_on = tid < A_CH;  // only matters when the A stage has < 256 chunks

  uint4 ra[A_PT], rb[B_PT];
  float rs[B_PT];
#define MLS_WQ_LOAD(k0)                                                                          \
  {                                                                                              \
    _Pragma("unroll") for (int i = 0; i < A_PT; ++i) if (A_CH >= 256 || a_on) ra[i] =            \
        __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsa, a_off[i], (k0) * ESZ, 0)); \
    _Pragma("unroll") for (int i = 0; i < B_PT; ++i) {                                           \
      rb[i] = __builtin_bit_cast(uint4,                                                          \
          __builtin_amdgcn_raw_buffer_load_b128(rsb, b_off[i], (k0) * WBITS / 8, 0));            \
      if constexpr (WBITS == 4)                                                                  \
        rs[i] = scale_at(s, s_dt, b_srow[i] + (int64_t)(((k0) + b_cc * KPC) / group) * ld_sg);   \
    }                                                                                            \
  }
#define MLS_WQ_STORE(buf)                                                                        \
  {                                                                                              \
    uint4* as_ = As + (buf) * BM * 8;                                                            \
    uint4* bs_ = Bs + (buf) * BN * 8;                                                            \
    _Pragma("unroll") for (int i = 0; i < A_PT; ++i) if (A_CH >= 256 || a_on)                    \
        as_[a_lds0 + 256 * i] = ra[i];                                                           \
    _Pragma("unroll") for (int i = 0; i < B_PT; ++i) {                                           \
      const int row = b_row0 + RSTEP * i;                                                        \
      if constexpr (WBITS == 8) {                                                                \
        uint32_t o[8];                                                                           \
        deq_int8<AT>(rb[i], o);                                                                  \
        const int c0 = b_cc * 2; /* 16 k -> two 8-k LDS chunks */                                \
        bs_[row * 8 + ((c0 + 0) ^ (row & 7))] = make_uint4(o[0], o[1], o[2], o[3]);             \
        bs_[row * 8 + ((c0 + 1) ^ (row & 7))] = make_uint4(o[4], o[5], o[6], o[7]);             \
      } else {                                                                                   \
        uint32_t o[16];                                                                          \
        deq_int4<AT>(rb[i], rs[i], o);                                                           \
        const int c0 = b_cc * 4; /* 32 k -> four 8-k LDS chunks */                               \
        _Pragma("unroll") for (int h = 0; h < 4; ++h)                                            \
          bs_[row * 8 + ((c0 + h) ^ (row & 7))] =                                                \
              make_uint4(o[4 * h + 0], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);                \
      }                                                                                          \
    }                                                                                            \
  }

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = K / BK;
  MLS_WQ_LOAD(0)
  MLS_WQ_STORE(0)
  __syncthreads();

  const int lr = lane & 15, lk = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) MLS_WQ_LOAD((kt + 1) * BK)
    const uint4* as = As + buf * BM * 8;
    const uint4* bs = Bs + buf * BN * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = ks * 4 + lk;
      uint4 bop[TN], aop[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int row = wn0 + i * 16 + lr;
        bop[i] = bs[row * 8 + (ch ^ (row & 7))];
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int row = wm0 + j * 16 + lr;
        aop[j] = as[row * 8 + (ch ^ (row & 7))];
      }
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = Mfma16<AT>::mma(bop[i], aop[j], acc[i][j]);
    }
    if (kt + 1 < nk) MLS_WQ_STORE(buf ^ 1)
    __syncthreads();
  }

#undef MLS_WQ_LOAD
#undef MLS_WQ_STORE

  // ---- epilogue: lane holds n = .. + 4*lk + r (r = 0..3), m = .. + lr
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nb = n0 + wn0 + i * 16 + 4 * lk;
    float sn[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (WBITS == 8) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sn[r] = nb + r < N ? scale_at(s, s_dt, nb + r) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int m = m0 + wm0 + j * 16 + lr;
      if (m >= row_hi) continue;
      AT* dst = c + (int64_t)m * ldc + nb;
      if (nb + 3 < N && (ldc % 4) == 0) {
        store4<AT>(dst, acc[i][j][0] * sn[0], acc[i][j][1] * sn[1], acc[i][j][2] * sn[2],
                   acc[i][j][3] * sn[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) dst[r] = from_f32<AT>(acc[i][j][r] * sn[r]);
      }
    }
  }
}

template <int WBITS, typename AT, int BM, int BN, int WM, int WN, bool GROUPED>
static int launch_tile(const WqArgs& p, int m_tiles, const int32_t* seg_off, int E,
                       int64_t w_estride, int64_t s_estride) {
  const int n_tiles = (int)cdiv(p.N, BN);
  const size_t lds = (size_t)2 * (BM + BN) * 64 * 2;
  auto kern = gemm_wq_mfma_kernel<WBITS, AT, BM, BN, WM, WN, GROUPED>;
  static bool attr_set = false;  // raise the dynamic LDS limit once per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(MLS_ERR_HIP, "gemm_wq_mfma: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  const int64_t blocks = (int64_t)n_tiles * m_tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), lds, p.stream, (const AT*)p.a, p.lda,
                     p.w, p.ldw, p.s, p.s_dt, p.ld_sn, p.ld_sg, p.group, (AT*)p.c, p.ldc, (int)p.M,
                     (int)p.N, (int)p.K, n_tiles, m_tiles, seg_off, E, w_estride, s_estride);
  return check_launch("gemm_wq_mfma");
}

// Tile choice for the dense GEMM: the tile shape whose (rounds of 256 blocks) x
// (tile area) is smallest, i.e. the least padded MFMA work once the last
// partial round is counted.
template <int WBITS, typename AT>
static int dense_dispatch(const WqArgs& p) {
  const int64_t nt = cdiv(p.N, 256);
  struct Cand { int bm; };
  const int bms[5] = {256, 128, 64, 32, 16};
  int best = 16;
  double best_cost = 1e300;
  for (int bm : bms) {
    if (bm > 16 && p.M <= bm / 2) continue;  // a smaller tile covers M
    const int64_t tiles = nt * cdiv(p.M, bm);
    const double cost = (double)cdiv(tiles, 256) * bm * 256.0;
    if (cost < best_cost * 0.999) { best_cost = cost; best = bm; }
  }
  const int mt = (int)cdiv(p.M, best);
  switch (best) {
    case 256: return launch_tile<WBITS, AT, 256, 256, 2, 2, false>(p, mt, nullptr, 0, 0, 0);
    case 128: return launch_tile<WBITS, AT, 128, 256, 2, 2, false>(p, mt, nullptr, 0, 0, 0);
    case 64: return launch_tile<WBITS, AT, 64, 256, 1, 4, false>(p, mt, nullptr, 0, 0, 0);
    case 32: return launch_tile<WBITS, AT, 32, 256, 1, 4, false>(p, mt, nullptr, 0, 0, 0);
    default: return launch_tile<WBITS, AT, 16, 256, 1, 4, false>(p, mt, nullptr, 0, 0, 0);
  }
}

// The kernels address one 256-row tile of each operand through a 32-bit buffer
// descriptor.
static bool tile_bytes_fit(const WqArgs& p) {
  return p.lda * dt_size(p.a_dt) * 256 < (1ll << 31) && p.ldw * 256 < (1ll << 31);
}

int launch_gemm_wq_mfma(int wbits, const WqArgs& p) {
  if (p.a_dt != MLS_F16 && p.a_dt != MLS_BF16) return MLS_ERR_UNSUPPORTED;
  if (p.K % 64 != 0) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && p.group % 32 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || p.lda % 8 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.c, 8)) return MLS_ERR_UNSUPPORTED;
  if (p.M > 0x3FFFFFFF || p.N > 0x3FFFFFFF || p.K > 0x3FFFFFFF) return MLS_ERR_UNSUPPORTED;
  if (!tile_bytes_fit(p)) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4)
    return p.a_dt == MLS_BF16 ? dense_dispatch<4, __bf16>(p) : dense_dispatch<4, _Float16>(p);
  return p.a_dt == MLS_BF16 ? dense_dispatch<8, __bf16>(p) : dense_dispatch<8, _Float16>(p);
}

int launch_grouped_int4(const GroupedArgs& g) {
  const WqArgs& p = g.base;
  if (p.a_dt != MLS_F16 && p.a_dt != MLS_BF16) return MLS_ERR_UNSUPPORTED;
  if (p.K % 64 != 0 || p.group % 32 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || p.lda % 8 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0 || g.w_estride % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.c, 8)) return MLS_ERR_UNSUPPORTED;
  if (!tile_bytes_fit(p)) return MLS_ERR_UNSUPPORTED;
  constexpr int BM = 128;
  // upper bound on sum_e ceil(rows_e / BM), without reading the device offsets
  const int m_tiles = (int)(cdiv(p.M, BM) + g.E);
  if (p.a_dt == MLS_BF16)
    return launch_tile<4, __bf16, BM, 256, 2, 2, true>(p, m_tiles, g.seg_off, g.E, g.w_estride,
                                                       g.s_estride);
  return launch_tile<4, _Float16, BM, 256, 2, 2, true>(p, m_tiles, g.seg_off, g.E, g.w_estride,
                                                       g.s_estride);
}

}  // namespace mls
