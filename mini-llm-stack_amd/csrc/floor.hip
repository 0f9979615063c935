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
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(256) void floor_empty_kernel() {}

__global__ __launch_bounds__(64) void floor_stamp_kernel(uint64_t* out) {
  if (threadIdx.x == 0) *out = __builtin_amdgcn_s_memrealtime();
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Wavefront w of the grid reads the contiguous chunks [w * per_wave, (w + 1) * per_wave):
// each load instruction covers 1 KiB, and all L loads of a lane are issued before any
// is used, as in the GEMV (one wavefront per SIMD, 256 blocks for the headline).
template <int L, bool STORE>
__global__ __launch_bounds__(256) void floor_stream_kernel(const u32x4_t* __restrict__ buf, int64_t chunks,
                                                           int64_t per_wave, uint32_t* __restrict__ sink) {
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
static int stream(const void* buf, int64_t bytes, int blocks, uint32_t* sink, hipStream_t st, bool store) {
  if (!buf || !sink || bytes <= 0 || bytes % 16 != 0 || blocks < 1) return -1;
  const int64_t chunks = bytes / 16;
  const int64_t per_wave = (chunks + 4LL * blocks - 1) / (4LL * blocks);
  const int64_t lpl = (per_wave + 63) / 64;
  const auto* p = static_cast<const u32x4_t*>(buf);
  const dim3 g((unsigned)blocks), b(256);
  switch (lpl) {
#define MLSF_L(L_)                                                                               \
  case L_:                                                                                       \
    if (store)                                                                                   \
      hipLaunchKernelGGL((floor_stream_kernel<L_, true>), g, b, 0, st, p, chunks, per_wave, sink);  \
    else                                                                                         \
      hipLaunchKernelGGL((floor_stream_kernel<L_, false>), g, b, 0, st, p, chunks, per_wave, sink); \
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
