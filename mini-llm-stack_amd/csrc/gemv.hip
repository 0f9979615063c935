// Decode-shaped weight-only GEMM (small M): the HBM-bound family. The lane layout, the
// dequantising dot products and the M = 1 kernel's body are in gemv1.h.
#include <type_traits>

#include "gemv1.h"

namespace mls {

// Every load is unconditional: indices past the matrix are clamped to valid rows
// and chunks, so the loads are independent and all issue before the first wait.
// Chunks past K contribute nothing (their term is selected away); rows past N or
// M are computed on clamped data and never stored.
template <int WBITS, typename AT, typename ST, int MT, int CPL, int R>
// Arguments for kernel-argument preloading (the first 14 dwords arrive in SGPRs): what the
// loads need first, strides as 32-bit values (launch_gemv_wq checks that they fit), the
// output last.
__global__ __launch_bounds__(256) void gemv_wq_kernel(
    const AT* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ s, int K, int N, int M,
    int ldx32, int ldw32, int ld_sn32, int ld_sg32, int group, AT* __restrict__ y, int64_t ldy) {
  const int64_t ldx = ldx32, ldw = ldw32, ld_sn = ld_sn32, ld_sg = ld_sg32;
  using S = XSlot<WBITS, AT>;
  constexpr int KC = S::KC, NV = S::NV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunks = K / KC;
  const int m0 = blockIdx.y * MT;
  const int n0 = (blockIdx.x * 4 + wave) * R;

  // 1. the lane's raw x pieces for MT rows first (L2 hits): vector loads complete in
  //    issue order, so unpacking x below waits for x only, and the dot product of a
  //    weight chunk waits only for that chunk, overlapping the arrival of the rest
  XRaw<WBITS, AT> xraw[MT][CPL];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const AT* xrow = x + (int64_t)min(m0 + mi, M - 1) * ldx;
#pragma unroll
    for (int j = 0; j < CPL; ++j) load_x_raw<WBITS, AT>(xrow, min(lane + 64 * j, nchunks - 1), xraw[mi][j]);
  }

  // 2. every weight chunk (and INT4 group scale) of this lane, in the order used
  //    (non-temporal: every weight byte is used once)
  uint4 wv[R][CPL];
  float sc[R][CPL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = min(n0 + r, N - 1);
    const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(w + n * ldw);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = min(lane + 64 * j, nchunks - 1);
      if constexpr (WBITS == 4)
        sc[r][j] = scale_value(s, n * ld_sn + (int64_t)((c * KC) / group) * ld_sg);
      const u32x4_t v = __builtin_nontemporal_load(wrow + c);
      wv[r][j] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads above are issued before any wait below

  uint32_t xr[MT][CPL][NV];
  float osx[MT][CPL];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int j = 0; j < CPL; ++j) osx[mi][j] = offset_term<WBITS, AT>(x_from_raw<WBITS, AT>(xraw[mi][j], xr[mi][j]));

  // 3. dot products. The INT4 16-bit path's widening constants live in VGPRs (an empty
  // asm hides their values, so they are not re-materialised as literals; see and_or).
  uint32_t nib_mask = 0x000F000Fu, magic = 0;
  if constexpr (WBITS == 4 && !S::F32) magic = Half16<AT>::MAGIC4;
  asm volatile("" : "+v"(nib_mask), "+v"(magic));
  float part[MT * R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        float d = chunk_dot<WBITS, AT>(wv[r][j], xr[mi][j], nib_mask, magic) - osx[mi][j];
        if (64 * (j + 1) > nchunks && lane + 64 * j >= nchunks) d = 0.0f;  // past K
        if constexpr (WBITS == 4) acc = fmaf(sc[r][j], d, acc);
        else acc += d;
      }
      part[mi * R + r] = acc;
    }
  }

  // 4. reduce all MT*R partials across the wavefront at once; lane L then holds
  //    the total of partial L / (64 / (MT*R))
  constexpr int V = MT * R;
  wave_reduce_many<V>(part);
  if (lane % (64 / V) == 0) {
    const int idx = lane / (64 / V);
    const int mi = idx / R, r = idx % R;
    const int m = m0 + mi, n = n0 + r;
    if (m < M && n < N) {
      float v = part[0];
      if constexpr (WBITS == 8) v *= scale_value(s, n);
      y[(int64_t)m * ldy + n] = from_f32<AT>(v);
    }
  }
}

// M = 1 (and M = 2) with 16-bit activations: x and the group scales through LDS (gemv1.h).
// This file is built with kernel-argument preloading: the first 14 dwords of the arguments
// arrive in SGPRs at wavefront start. They hold everything the kernel needs before its
// weight loads, so no load waits for a scalar load of the arguments (the output pointer and
// stride come last). The weight buffer's size is N ldw (as the 32-bit product), and the
// launcher takes MX = M.
template <int WBITS, typename AT, typename ST, int CPL, int R, int XI, int SI, int MX>
__global__ __launch_bounds__(256) void gemv1_kernel(const AT* __restrict__ x, const uint8_t* __restrict__ w,
                                                    const ST* __restrict__ s, int K, int N, int ldw, int s_bytes,
                                                    int s_dw, int s_row_bytes, int group, int lda_b,
                                                    AT* __restrict__ y, int ldy) {
  const int w_bytes = (int)((uint32_t)N * (uint32_t)ldw);
  gemv1_body<WBITS, AT, ST, CPL, R, XI, SI, MX>(x, w, ldw, w_bytes, s, s_row_bytes, s_bytes, group, y, N, K, s_dw,
                                                lda_b, MX, ldy);
}

template <int WBITS, typename AT, typename ST, int CPL, int SI>
static int launch_gemv1_si(const WqArgs& p, int s_dw) {
  constexpr int R2 = CPL >= 8 ? 1 : 8 / CPL;  // rows per wavefront: 8 loads per lane
  // x instructions per wavefront: 4 wavefronts x 1 KiB cover the K sizeof(AT) bytes of x
  // (16-bit x: INT4 K <= 2048 CPL, INT8 K <= 1024 CPL; fp32 x twice the instructions)
  constexpr int XI16 = WBITS == 4 ? CPL : (CPL >= 2 ? CPL / 2 : 1);
  constexpr int XI = std::is_same_v<AT, float> ? 2 * XI16 : XI16;
  if (p.K * (int64_t)sizeof(AT) > XI * 4096) return MLS_ERR_UNSUPPORTED;
  const int s_row_bytes = (int)(p.ld_sn * (int64_t)sizeof(ST));
  // the scale descriptor spans exactly the scales that exist: row N - 1 starts at
  // (N - 1) ld_sn and holds G groups (ld_sn may be below G, e.g. 0 for one row broadcast)
  const int s_bytes =
      WBITS == 4 ? (int)(((p.N - 1) * p.ld_sn + p.K / p.group) * (int64_t)sizeof(ST)) : 0;
  // rows of x: 1 or 2 (3 and 4 rows measured slower than the MFMA skinny kernel: the dot
  // products grow with M while the widening is shared); x of both rows in LDS within 32 KiB
  if (p.M > 2) return MLS_ERR_UNSUPPORTED;
  const int mx = (int)p.M;
  const int64_t lda_b = p.lda * (int64_t)sizeof(AT);
  if (mx > 1 && (mx * XI > 8 || (p.M - 1) * lda_b + p.K * (int64_t)sizeof(AT) > 0x7FFFFFFF))
    return MLS_ERR_UNSUPPORTED;
  auto go = [&](auto mxc, auto rc) {
    constexpr int MX = decltype(mxc)::value, R = decltype(rc)::value;
    hipLaunchKernelGGL((gemv1_kernel<WBITS, AT, ST, CPL, R, XI, SI, MX>), dim3((unsigned)cdiv(p.N, 4 * R)), dim3(256),
                       0, p.stream, (const AT*)p.a, p.w, (const ST*)p.s, (int)p.K, (int)p.N, (int)p.ldw, s_bytes,
                       s_dw, s_row_bytes, p.group, (int)(mx > 1 ? lda_b : 0), (AT*)p.c, (int)(mx > 1 ? p.ldc : 0));
    return MLS_OK;
  };
  using I1 = std::integral_constant<int, 1>;
  if (mx == 1) {
    // INT8 with one row of x: half the rows per wavefront, twice the wavefronts (K = 2048:
    // 2.82 -> 2.72 us; K = 4096 the same; with two rows of x it measured 4% slower)
    if constexpr (WBITS == 8) return go(I1{}, std::integral_constant<int, (CPL >= 4 ? 1 : 4 / CPL)>{});
    // INT4 with K <= 2048 (8 rows per wavefront): 2 rows when 8 would leave CUs without a
    // block (the reference's bench shape, N = K = 2048 g64: 64 -> 256 blocks, 3.54 -> 2.71 us)
    if constexpr (WBITS == 4 && CPL == 1)
      if (p.N < 4 * R2 * 256) return go(I1{}, std::integral_constant<int, 2>{});
    return go(I1{}, std::integral_constant<int, R2>{});
  }
  if constexpr (XI <= 4 && !std::is_same_v<AT, float>)
    return go(std::integral_constant<int, 2>{}, std::integral_constant<int, R2>{});
  return MLS_ERR_UNSUPPORTED;
}

template <int WBITS, typename AT, typename ST, int CPL>
static int launch_gemv1_cpl(const WqArgs& p, int s_dw) {
  constexpr int R = CPL >= 8 ? 1 : 8 / CPL;
  if constexpr (WBITS == 8) return launch_gemv1_si<WBITS, AT, ST, CPL, 1>(p, s_dw);
  const int64_t slice = (int64_t)R * s_dw;  // scale dwords per wavefront
  if (slice <= 64) return launch_gemv1_si<WBITS, AT, ST, CPL, 1>(p, s_dw);
  if (slice <= 128) return launch_gemv1_si<WBITS, AT, ST, CPL, 2>(p, s_dw);
  if (slice <= 256) return launch_gemv1_si<WBITS, AT, ST, CPL, 4>(p, s_dw);
  return MLS_ERR_UNSUPPORTED;
}

template <int WBITS, typename AT, typename ST>
static int launch_gemv1_st(const WqArgs& p) {
  constexpr int KC = XSlot<WBITS, AT>::KC;
  int s_dw = 0;
  if constexpr (WBITS == 4) {
    const int64_t G = p.K / p.group;
    // group scales read as whole dwords per row: contiguous groups, rows on dword boundaries
    if (p.ld_sg != 1 || (G * (int64_t)sizeof(ST)) % 4 != 0 || (p.ld_sn * (int64_t)sizeof(ST)) % 4 != 0 ||
        !aligned(p.s, 4))
      return MLS_ERR_UNSUPPORTED;
    if (((int64_t)p.N * p.ld_sn + G) * (int64_t)sizeof(ST) > 0x7FFFFFFF) return MLS_ERR_UNSUPPORTED;
    s_dw = (int)(G * (int64_t)sizeof(ST) / 4);
  }
  const int64_t cpl = cdiv(p.K / KC, 64);
  if (cpl <= 1) return launch_gemv1_cpl<WBITS, AT, ST, 1>(p, s_dw);
  if (cpl <= 2) return launch_gemv1_cpl<WBITS, AT, ST, 2>(p, s_dw);
  if (cpl <= 4) return launch_gemv1_cpl<WBITS, AT, ST, 4>(p, s_dw);
  if (cpl <= 8) return launch_gemv1_cpl<WBITS, AT, ST, 8>(p, s_dw);
  if constexpr (WBITS == 8)  // (INT4 with 16 chunks per lane has K > 16384: x would not fit)
    if (cpl <= 16) return launch_gemv1_cpl<WBITS, AT, ST, 16>(p, s_dw);
  return MLS_ERR_UNSUPPORTED;
}

// M = 1 (and, through launch_gemv_rows, M = 2) with 16-bit activations;
// MLS_ERR_UNSUPPORTED sends the call to gemv_wq_kernel. MLS_GEMV1=0 disables this path
// (A/B sweeps).
static int launch_gemv1(int wbits, const WqArgs& p) {
  static const int enabled = env_int("MLS_GEMV1", 1);
  // fp32 x with M = 1, INT4: x split into bf16 hi + lo parts (K = N = 4096 g128: 4.98 -> 4.27 us
  // against the register kernel; INT8 measured slower that way, 5.64 -> 6.06, and keeps the
  // register kernel). MLS_GEMV1_F32=0: the register kernel for INT4 too (A/B runs).
  static const int f32_on = env_int("MLS_GEMV1_F32", 1);
  if (!enabled || p.M < 1 || p.M > 2 || (p.a_dt == MLS_F32 && (p.M != 1 || !f32_on || wbits != 4)))
    return MLS_ERR_UNSUPPORTED;
  // x in LDS (at most 32 KiB); 32-bit buffer offsets into the whole weight matrix
  if (p.K * dt_size(p.a_dt) > 32768 || (p.N + 4) * p.ldw >= (1ll << 31)) return MLS_ERR_UNSUPPORTED;
  if (p.a_dt == MLS_F32)
    return p.s_dt == MLS_F16 ? launch_gemv1_st<4, float, _Float16>(p) : launch_gemv1_st<4, float, float>(p);
  if (wbits == 4) {
    if (p.a_dt == MLS_F16) return p.s_dt == MLS_F16 ? launch_gemv1_st<4, _Float16, _Float16>(p)
                                                    : launch_gemv1_st<4, _Float16, float>(p);
    return p.s_dt == MLS_F16 ? launch_gemv1_st<4, __bf16, _Float16>(p) : launch_gemv1_st<4, __bf16, float>(p);
  }
  if (p.a_dt == MLS_F16) return p.s_dt == MLS_F16 ? launch_gemv1_st<8, _Float16, _Float16>(p)
                                                  : launch_gemv1_st<8, _Float16, float>(p);
  return p.s_dt == MLS_F16 ? launch_gemv1_st<8, __bf16, _Float16>(p) : launch_gemv1_st<8, __bf16, float>(p);
}

template <int WBITS, typename AT, typename ST, int MT, int CPL, int R>
static void launch_r(const WqArgs& p) {
  const dim3 grid((unsigned)cdiv(p.N, 4 * R), (unsigned)cdiv(p.M, MT));
  hipLaunchKernelGGL((gemv_wq_kernel<WBITS, AT, ST, MT, CPL, R>), grid, dim3(256), 0, p.stream,
                     (const AT*)p.a, p.w, (const ST*)p.s, (int)p.K, (int)p.N, (int)p.M, (int)p.lda, (int)p.ldw,
                     (int)p.ld_sn, (int)p.ld_sg, p.group, (AT*)p.c, p.ldc);
}

// Rows per wavefront: by default enough that each lane has 8 weight chunks in
// flight (R * CPL = 8); MLS_GEMV_ROWS (1, 2, 4 or 8) overrides it for tuning.
static int gemv_rows_override() {
  static const int v = [] {
    const char* e = getenv("MLS_GEMV_ROWS");
    const int r = e ? atoi(e) : 0;
    return (r == 1 || r == 2 || r == 4 || r == 8) ? r : 0;
  }();
  return v;
}

// Overrides stay within R * CPL <= 16 chunks per lane and MT * R <= 32 (beyond that the
// kernel spills).
template <int WBITS, typename AT, typename ST, int MT, int CPL>
static void launch_one(const WqArgs& p) {
  constexpr int RDEF = CPL >= 8 ? 1 : 8 / CPL;
  int r = gemv_rows_override();
  if (r == 0 || MT * r > 32 || r * CPL > 16) r = RDEF;
  switch (r) {
    case 1: return launch_r<WBITS, AT, ST, MT, CPL, 1>(p);
    case 2:
      if constexpr (2 * CPL <= 16) return launch_r<WBITS, AT, ST, MT, CPL, 2>(p);
      break;
    case 4:
      if constexpr (4 * CPL <= 16 && MT * 4 <= 32) return launch_r<WBITS, AT, ST, MT, CPL, 4>(p);
      break;
    default:
      if constexpr (8 * CPL <= 16 && MT * 8 <= 32) return launch_r<WBITS, AT, ST, MT, CPL, 8>(p);
      break;
  }
  return launch_r<WBITS, AT, ST, MT, CPL, RDEF>(p);
}

// Picks MT (rows of x per block) for a given CPL so that the x slice fits in
// 128 registers: MT * CPL * NV <= 128.
template <int WBITS, typename AT, typename ST, int CPL>
static int dispatch_mt(const WqArgs& p) {
  constexpr int NV = XSlot<WBITS, AT>::NV;
  constexpr int MAXMT = 128 / (CPL * NV);
  if constexpr (MAXMT < 1) {
    return MLS_ERR_UNSUPPORTED;
  } else {
    if (p.M == 1 || MAXMT < 2) launch_one<WBITS, AT, ST, 1, CPL>(p);
    else if (p.M == 2 || MAXMT < 4) launch_one<WBITS, AT, ST, (MAXMT >= 2 ? 2 : 1), CPL>(p);
    else launch_one<WBITS, AT, ST, (MAXMT >= 4 ? 4 : 1), CPL>(p);
    return MLS_OK;
  }
}

template <int WBITS, typename AT, typename ST>
static int dispatch_cpl(const WqArgs& p) {
  constexpr int KC = XSlot<WBITS, AT>::KC;
  const int64_t cpl = cdiv(p.K / KC, 64);
  if (cpl <= 1) return dispatch_mt<WBITS, AT, ST, 1>(p);
  if (cpl <= 2) return dispatch_mt<WBITS, AT, ST, 2>(p);
  if (cpl <= 4) return dispatch_mt<WBITS, AT, ST, 4>(p);
  if (cpl <= 8) return dispatch_mt<WBITS, AT, ST, 8>(p);
  if (cpl <= 16) return dispatch_mt<WBITS, AT, ST, 16>(p);
  return MLS_ERR_UNSUPPORTED;
}

template <int WBITS, typename AT>
static int dispatch_st(const WqArgs& p) {
  return p.s_dt == MLS_F16 ? dispatch_cpl<WBITS, AT, _Float16>(p) : dispatch_cpl<WBITS, AT, float>(p);
}

int launch_gemv_wq(int wbits, const WqArgs& p) {
  const int KC = wbits == 4 ? 32 : 16;
  const int esz = dt_size(p.a_dt);
  if (p.K % KC != 0) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && (p.group % KC != 0)) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || (p.lda * esz) % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (p.N > 0x7FFFFFFF / 2 || p.M > 4 * 65535) return MLS_ERR_UNSUPPORTED;  // grid.y = M / MT
  const int rc = p.M == 1 ? launch_gemv1(wbits, p) : MLS_ERR_UNSUPPORTED;
  if (rc != MLS_ERR_UNSUPPORTED) return rc;
  // gemv_wq_kernel takes the strides as 32-bit arguments
  if (p.lda > 0x7FFFFFFF || p.ldw > 0x7FFFFFFF || p.ld_sn > 0x7FFFFFFF || p.ld_sg > 0x7FFFFFFF)
    return MLS_ERR_UNSUPPORTED;
  if (wbits == 4) {
    if (p.a_dt == MLS_F32) return dispatch_st<4, float>(p);
    if (p.a_dt == MLS_F16) return dispatch_st<4, _Float16>(p);
    return dispatch_st<4, __bf16>(p);
  }
  if (p.a_dt == MLS_F32) return dispatch_st<8, float>(p);
  if (p.a_dt == MLS_F16) return dispatch_st<8, _Float16>(p);
  return dispatch_st<8, __bf16>(p);
}

// M = 2 on the M = 1 kernel's layout (every weight chunk widened once, dotted with
// each row of x); MLS_ERR_UNSUPPORTED when the shape or alignment does not fit it.
int launch_gemv_rows(int wbits, const WqArgs& p) {
  const int KC = wbits == 4 ? 32 : 16;
  if (p.M != 2 || p.a_dt == MLS_F32 || p.K % KC != 0) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && (p.group % KC != 0)) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || (p.lda * 2) % 16 != 0 || p.N > 0x7FFFFFFF / 2) return MLS_ERR_UNSUPPORTED;
  return launch_gemv1(wbits, p);
}

// ------------------------------------------------------------------ generic path

template <int WBITS, typename AT>
__global__ void gemm_wq_generic_kernel(const AT* __restrict__ x, int64_t ldx,
                                       const uint8_t* __restrict__ w, int64_t ldw,
                                       const void* __restrict__ s, int s_dt, int64_t ld_sn,
                                       int64_t ld_sg, int group, AT* __restrict__ y, int64_t ldy,
                                       int64_t M, int64_t N, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * N) return;
  const int64_t m = t / N, n = t - m * N;
  const AT* xr = x + m * ldx;
  const uint8_t* wr = w + n * ldw;
  float acc = 0.0f;
  if constexpr (WBITS == 8) {
    for (int64_t k = 0; k < K; ++k) acc = fmaf(to_f32(xr[k]), (float)(int8_t)wr[k], acc);
    acc *= load_scale(s, s_dt, n);
  } else {
    for (int64_t k = 0; k < K; ++k) {
      const uint32_t byte = wr[k >> 1];
      const uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 15u);
      const float wk = ((float)nib - 8.0f) * load_scale(s, s_dt, n * ld_sn + (k / group) * ld_sg);
      acc = fmaf(to_f32(xr[k]), wk, acc);
    }
  }
  y[m * ldy + n] = from_f32<AT>(acc);
}

int launch_gemm_wq_generic(int wbits, const WqArgs& p) {
  const int64_t work = p.M * p.N;
  const dim3 grid((unsigned)cdiv(work, 256));
#define MLS_GENERIC(WB, T)                                                                        \
  hipLaunchKernelGGL((gemm_wq_generic_kernel<WB, T>), grid, dim3(256), 0, p.stream,              \
                     (const T*)p.a, p.lda, p.w, p.ldw, p.s, p.s_dt, p.ld_sn, p.ld_sg, p.group,    \
                     (T*)p.c, p.ldc, p.M, p.N, p.K)
  if (wbits == 4) {
    if (p.a_dt == MLS_F32) MLS_GENERIC(4, float);
    else if (p.a_dt == MLS_F16) MLS_GENERIC(4, _Float16);
    else MLS_GENERIC(4, __bf16);
  } else {
    if (p.a_dt == MLS_F32) MLS_GENERIC(8, float);
    else if (p.a_dt == MLS_F16) MLS_GENERIC(8, _Float16);
    else MLS_GENERIC(8, __bf16);
  }
#undef MLS_GENERIC
  return MLS_OK;
}

}  // namespace mls
