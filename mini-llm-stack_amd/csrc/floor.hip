// Calibration kernels for the single-launch floor of bench.py's M = 1 GEMV rows. They are
// not part of the library or its ABI (built into their own libmls_floor.so, loaded only
// by bench.py): they bound what one launch of the headline's size can reach on this GPU.
//
//   mlsf_empty:  a kernel that does nothing, launched with the GEMV's grid: the cost of a
//                launch in a HIP graph.
//   mlsf_stream: a streaming read of `bytes` with the GEMV's geometry (16-byte
//                non-temporal loads, no arithmetic beyond an xor of what was read, which is
//                stored only if it equals a value the data does not hold, so the loads are
//                not removed): the most a single launch can move through HBM at this size.
//   mlsf_stream_store: the same read, and every wavefront then stores 8 bytes (the xor,
//                twice) as the GEMV's wavefronts store their 4 outputs: the read plus the
//                cost of a kernel that writes its result.
//   mlsf_stamp:  one thread stores the GPU's constant-rate realtime counter
//                (s_memrealtime, mlsf_wallclock_khz ticks per millisecond) with an
//                ordinary vector store. bench.py captures one before and one after the
//                timed steps inside the graph that also holds the warmup steps, so the
//                graph's own launch cost (paid before its first node) stays outside the
//                interval.
//
// Clocked copies (timing only): the library's M = 1 GEMV kernel body (gemv1.h, the same
// force-inlined device code the library's gemv1_kernel runs) and the kernels above, with
// every wavefront reading the realtime counter at its first instruction (t0) and again
// at its end (t1), then storing {t0, t1} with one 16-byte vector store at clocks[2 w] for
// its flat wavefront index w. Two ends (`wait`): 0, right after the wavefront's last
// instruction issued (every load has returned, since every result was used; its output
// store may still be in flight), or 1, after all of its memory operations completed
// (behind an s_waitcnt of every counter, which keeps the wavefront alive until its
// stores are acknowledged). min t0 .. max t1 over a launch is its execution span on
// the GPU, without the profiler and without the launch and completion processing
// around it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv1.h"

namespace {

// {t0, t1} of this wavefront; t0 was read before anything else the kernel did
template <bool WAIT>
__device__ __forceinline__ void store_clocks(uint64_t* __restrict__ clocks, uint64_t t0) {
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (WAIT) {
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt, expcnt, lgkmcnt all zero: loads, LDS and stores done
    __builtin_amdgcn_sched_barrier(0);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
  if ((threadIdx.x & 63) == 0) {
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    reinterpret_cast<ulonglong2*>(clocks)[w] = make_ulonglong2(t0, t1);
  }
}

__global__ __launch_bounds__(256) void floor_empty_clocked_kernel(uint64_t* __restrict__ clocks) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  store_clocks<false>(clocks, t0);
}

__global__ __launch_bounds__(256) void floor_empty_kernel() {}

__global__ __launch_bounds__(64) void floor_stamp_kernel(uint64_t* out) {
  if (threadIdx.x == 0) *out = __builtin_amdgcn_s_memrealtime();
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Wavefront w of the grid reads the contiguous chunks [w * per_wave, (w + 1) * per_wave):
// each load instruction covers 1 KiB, and all L loads of a lane are issued before any
// is used, as in the GEMV (one wavefront per SIMD, 256 blocks for the headline).
template <int L, bool STORE, int CLOCK = 0>  // CLOCK: 0 none, 1 issue end, 2 memory end
__global__ __launch_bounds__(256) void floor_stream_kernel(const u32x4_t* __restrict__ buf, int64_t chunks,
                                                           int64_t per_wave, uint32_t* __restrict__ sink,
                                                           uint64_t* __restrict__ clocks = nullptr) {
  uint64_t t0 = 0;
  if constexpr (CLOCK != 0) {
    t0 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t c0 = w * per_wave;
  // unconditional loads (a chunk index past the span or the buffer is clamped: a few
  // chunks are read twice), so none waits behind a branch
  u32x4_t d[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int64_t c = c0 + min<int64_t>(64 * i + lane, per_wave - 1);
    d[i] = __builtin_nontemporal_load(buf + min<int64_t>(c, chunks - 1));
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before any is used
  uint32_t v = 0;
#pragma unroll
  for (int i = 0; i < L; ++i) v ^= d[i].x ^ d[i].y ^ d[i].z ^ d[i].w;
  if constexpr (STORE) {
    // lane 63 holds the wavefront's value after the same kind of cross-lane steps the
    // GEMV's reduction takes (one DPP row broadcast), and stores one 8-byte word per wavefront
    v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    if (lane == 63) reinterpret_cast<uint2*>(sink)[w] = make_uint2(v, v);
  } else {
    if (v == 0x9E3779B9u) sink[0] = v;
  }
  if constexpr (CLOCK != 0) store_clocks<CLOCK == 2>(clocks, t0);
}

// The library's M = 1 GEMV (gemv1.h) with 16-bit activations and fp16 scales, clocked.
template <int WBITS, typename AT, int CPL, int R, int XI, int SI, bool WAIT>
// Arguments in the library kernel's order (both files are built with kernel-argument preloading).
__global__ __launch_bounds__(256) void floor_gemv1_clocked_kernel(const AT* __restrict__ x,
                                                                  const uint8_t* __restrict__ w,
                                                                  const _Float16* __restrict__ s, int K, int N,
                                                                  int ldw, int s_bytes, int s_dw, int s_row_bytes,
                                                                  int group, AT* __restrict__ y,
                                                                  uint64_t* __restrict__ clocks) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  const int w_bytes = (int)((uint32_t)N * (uint32_t)ldw);
  mls::gemv1_body<WBITS, AT, _Float16, CPL, R, XI, SI, 1>(x, w, ldw, w_bytes, s, s_row_bytes, s_bytes, group, y,
                                                           N, K, s_dw, 0, 1, 0);
  store_clocks<WAIT>(clocks, t0);
}

}  // namespace

extern "C" int mlsf_empty(int blocks, hipStream_t st) {
  if (blocks < 1) return -1;
  hipLaunchKernelGGL(floor_empty_kernel, dim3((unsigned)blocks), dim3(256), 0, st);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// `blocks` blocks of 4 wavefronts share `bytes` (a multiple of 16) in equal contiguous
// spans; each lane issues up to 16 16-byte loads. store: `sink` holds 8 bytes per
// wavefront (blocks * 32 bytes), one word written by each.
static int stream(const void* buf, int64_t bytes, int blocks, uint32_t* sink, hipStream_t st, bool store,
                  uint64_t* clocks = nullptr, bool wait = false) {
  if (!buf || !sink || bytes <= 0 || bytes % 16 != 0 || blocks < 1) return -1;
  const int64_t chunks = bytes / 16;
  const int64_t per_wave = (chunks + 4LL * blocks - 1) / (4LL * blocks);
  const int64_t lpl = (per_wave + 63) / 64;
  const auto* p = static_cast<const u32x4_t*>(buf);
  const dim3 g((unsigned)blocks), b(256);
  switch (lpl) {
#define MLSF_L(L_)                                                                                           \
  case L_:                                                                                                   \
    if (clocks && store && wait)                                                                             \
      hipLaunchKernelGGL((floor_stream_kernel<L_, true, 2>), g, b, 0, st, p, chunks, per_wave, sink, clocks); \
    else if (clocks && store)                                                                                \
      hipLaunchKernelGGL((floor_stream_kernel<L_, true, 1>), g, b, 0, st, p, chunks, per_wave, sink, clocks); \
    else if (clocks && wait)                                                                                 \
      hipLaunchKernelGGL((floor_stream_kernel<L_, false, 2>), g, b, 0, st, p, chunks, per_wave, sink, clocks); \
    else if (clocks)                                                                                         \
      hipLaunchKernelGGL((floor_stream_kernel<L_, false, 1>), g, b, 0, st, p, chunks, per_wave, sink, clocks); \
    else if (store)                                                                                          \
      hipLaunchKernelGGL((floor_stream_kernel<L_, true>), g, b, 0, st, p, chunks, per_wave, sink);           \
    else                                                                                                     \
      hipLaunchKernelGGL((floor_stream_kernel<L_, false>), g, b, 0, st, p, chunks, per_wave, sink);          \
    break;
    MLSF_L(1) MLSF_L(2) MLSF_L(3) MLSF_L(4) MLSF_L(5) MLSF_L(6) MLSF_L(7) MLSF_L(8)
    MLSF_L(9) MLSF_L(10) MLSF_L(11) MLSF_L(12) MLSF_L(13) MLSF_L(14) MLSF_L(15) MLSF_L(16)
#undef MLSF_L
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int mlsf_stream(const void* buf, int64_t bytes, int blocks, uint32_t* sink, hipStream_t st) {
  return stream(buf, bytes, blocks, sink, st, false);
}

extern "C" int mlsf_stream_store(const void* buf, int64_t bytes, int blocks, uint32_t* sink, hipStream_t st) {
  return stream(buf, bytes, blocks, sink, st, true);
}

// Clocked copies: `clocks` receives 16 bytes per wavefront ({t0, t1}, realtime ticks);
// wait: 0 = t1 when the last instruction issued, 1 = after all memory operations completed.
extern "C" int mlsf_empty_clocked(int blocks, uint64_t* clocks, hipStream_t st) {
  if (blocks < 1 || !clocks) return -1;
  hipLaunchKernelGGL(floor_empty_clocked_kernel, dim3((unsigned)blocks), dim3(256), 0, st, clocks);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int mlsf_stream_clocked(const void* buf, int64_t bytes, int blocks, uint32_t* sink, int store,
                                   int wait, uint64_t* clocks, hipStream_t st) {
  if (!clocks) return -1;
  return stream(buf, bytes, blocks, sink, st, store != 0, clocks, wait != 0);
}

// The headline GEMVs exactly as the library launches them (the launch parameters of
// gemv.hip's launcher for these shapes): bf16 x [1][K], fp16 scales, K = 4096.
//   wbits 4: packed w [N][ldw] (ldw >= 2048), scales [N][ld_sn] with 32 groups of 128
//            (ld_sn >= 32, even); 4 rows per wavefront, 2 chunks per lane.
//   wbits 8: w [N][ldw] int8 (ldw >= 4096), scales [N]; 1 row per wavefront, 4 chunks per lane.
// Returns the number of wavefronts (the clocks written), or a negative code for any
// other shape, before anything is launched.
extern "C" int mlsf_gemv1_clocked(int wbits, const void* x, const uint8_t* w, int64_t ldw, const void* s,
                                  int64_t ld_sn, int group, void* y, int64_t N, int64_t K, int wait,
                                  uint64_t* clocks, hipStream_t st) {
  if (!x || !w || !s || !y || !clocks || K != 4096 || N < 1 || N > (1 << 20)) return -1;
  if ((N + 4) * ldw >= (1ll << 31)) return -1;
  if (wbits == 4) {
    if (group != 128 || ld_sn < 32 || ld_sn % 2 != 0 || ldw < 2048 || ldw % 16 != 0) return -1;
    const int blocks = (int)((N + 15) / 16);
    auto go = [&](auto wc) {
      hipLaunchKernelGGL((floor_gemv1_clocked_kernel<4, __bf16, 2, 4, 2, 1, decltype(wc)::value>),
                         dim3((unsigned)blocks), dim3(256), 0, st, (const __bf16*)x, w, (const _Float16*)s, (int)K,
                         (int)N, (int)ldw, (int)(((N - 1) * ld_sn + 32) * 2), 16, (int)(ld_sn * 2), group,
                         (__bf16*)y, clocks);
    };
    if (wait) go(std::true_type{});
    else go(std::false_type{});
    return hipGetLastError() == hipSuccess ? blocks * 4 : -2;
  }
  if (wbits == 8) {
    if (ldw < 4096 || ldw % 16 != 0) return -1;
    const int blocks = (int)((N + 3) / 4);
    auto go = [&](auto wc) {
      hipLaunchKernelGGL((floor_gemv1_clocked_kernel<8, __bf16, 4, 1, 2, 1, decltype(wc)::value>),
                         dim3((unsigned)blocks), dim3(256), 0, st, (const __bf16*)x, w, (const _Float16*)s, (int)K,
                         (int)N, (int)ldw, 0, 0, 2, 0, (__bf16*)y, clocks);
    };
    if (wait) go(std::true_type{});
    else go(std::false_type{});
    return hipGetLastError() == hipSuccess ? blocks * 4 : -2;
  }
  return -1;
}

extern "C" int mlsf_stamp(uint64_t* out, hipStream_t st) {
  if (!out) return -1;
  hipLaunchKernelGGL(floor_stamp_kernel, dim3(1), dim3(64), 0, st, out);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int mlsf_wallclock_khz(int* khz) {
  int dev = 0;
  if (!khz || hipGetDevice(&dev) != hipSuccess) return -1;
  return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess ? 0 : -2;
}
