// Internal helpers shared by the gfx950 kernels and the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../include/mls.h"

namespace mls {

// ----------------------------------------------------------------- host side

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks the launch that was just enqueued.
int check_launch(const char* what);

inline bool is_float_dt(int dt) { return dt == MLS_F32 || dt == MLS_F16 || dt == MLS_BF16; }
inline int dt_size(int dt) { return dt == MLS_F32 ? 4 : 2; }
inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
// integer value of a tuning environment variable (sweeps), dflt when unset or empty
inline int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

// ----------------------------------------------------------------- device side

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }

__device__ __forceinline__ uint32_t pack2_bits(__bf16 lo, __bf16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}
__device__ __forceinline__ uint32_t pack2_bits(_Float16 lo, _Float16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// Stores 4 consecutive outputs (converted from fp32) with one 8- or 16-byte store.
// dst must be aligned to 4 elements.
template <typename T>
__device__ __forceinline__ void store4(T* dst, float v0, float v1, float v2, float v3) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(dst) = make_float4(v0, v1, v2, v3);
  } else {
    const uint2 u = make_uint2(pack2_bits(from_f32<T>(v0), from_f32<T>(v1)),
                               pack2_bits(from_f32<T>(v2), from_f32<T>(v3)));
    *reinterpret_cast<uint2*>(dst) = u;
  }
}

// v moved across lanes by a DPP pattern (CTRL = dpp_ctrl encoding).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// v_permlane32_swap (BIT = 32) / v_permlane16_swap (BIT = 16): the lanes with lane & BIT
// of a trade places with the lanes without it of b (the upper 32 lanes of a with the lower
// 32 of b; the odd 16-lane rows of a with the even rows of b), so that a + b afterwards
// holds, in the lanes without the bit, a's value plus its xor-BIT partner's, and in the
// lanes with it, b's: the xor-shuffle step of a and b at once, without the LDS crossbar.
// The pair's elements are copied out one by one (a __builtin_bit_cast of the second
// element compiled into a read of the first).
template <int BIT>
__device__ __forceinline__ float swap_add(float a, float b) {
  static_assert(BIT == 16 || BIT == 32, "lane-half or 16-lane-row swap");
  uint32_t r0, r1;
  if constexpr (BIT == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    r0 = r[0];
    r1 = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    r0 = r[0];
    r1 = r[1];
  }
  return __uint_as_float(r0) + __uint_as_float(r1);
}

namespace detail {
// Halves the live values per step: lanes with lane & BIT keep the upper half,
// the others the lower half, each adding its xor-partner's copy. With one value
// left, the lane bits BIT..0 are summed (lowest first, so the mirror patterns
// pair lanes that already hold the sums of their quads / octets).
template <int N, int BIT>
__device__ __forceinline__ void reduce_split(float* v, int lane) {
  if constexpr (N > 1) {
    constexpr int H = N / 2;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      if constexpr (BIT >= 16) {
        v[i] = swap_add<BIT>(v[i], v[i + H]);
      } else {
        const bool upper = (lane & BIT) != 0;
        const float send = upper ? v[i] : v[i + H];
        const float keep = upper ? v[i + H] : v[i];
        v[i] = keep + __shfl_xor(send, BIT, 64);
      }
    }
    reduce_split<H, BIT / 2>(v, lane);
  } else {
    if constexpr (BIT >= 1) v[0] += dpp_mov<0xB1>(v[0]);   // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (BIT >= 2) v[0] += dpp_mov<0x4E>(v[0]);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (BIT >= 4) v[0] += dpp_mov<0x141>(v[0]);  // row_half_mirror: the other quad
    if constexpr (BIT >= 8) v[0] += dpp_mov<0x140>(v[0]);  // row_mirror: the other octet
    if constexpr (BIT >= 16) v[0] = swap_add<16>(v[0], v[0]);
    if constexpr (BIT >= 32) v[0] = swap_add<32>(v[0], v[0]);
  }
}
}  // namespace detail

// Sums V per-lane partials over the wavefront in one pass (V a power of two, <= 64).
// Afterwards v[0] of lane L holds the total of partial index L / (64 / V); the
// other entries of v are clobbered.
template <int V>
__device__ __forceinline__ void wave_reduce_many(float (&v)[V]) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
  detail::reduce_split<V, 32>(v, threadIdx.x & 63);
}

// Sum over each aligned group of W lanes (W a power of two, <= 64); every lane of a
// group receives its group's total, bit-identical to an xor-shuffle butterfly. After
// the two quad steps all lanes of a quad hold the same sum, so the mirror patterns
// fetch exactly the value the xor-4 / xor-8 partner holds.
template <int W>
__device__ __forceinline__ float lane_group_sum(float s) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "W must be a power of two <= 64");
  if constexpr (W >= 2) s += dpp_mov<0xB1>(s);   // lane ^ 1
  if constexpr (W >= 4) s += dpp_mov<0x4E>(s);   // lane ^ 2
  if constexpr (W >= 8) s += dpp_mov<0x141>(s);  // row_half_mirror: the other quad
  if constexpr (W >= 16) s += dpp_mov<0x140>(s); // row_mirror: the other octet
  if constexpr (W >= 32) s += __shfl_xor(s, 16, 64);
  if constexpr (W >= 64) s += __shfl_xor(s, 32, 64);
  return s;
}

// Maximum over each aligned group of W lanes, by the same pattern as lane_group_sum.
template <int W>
__device__ __forceinline__ float lane_group_max(float s) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "W must be a power of two <= 64");
  if constexpr (W >= 2) s = fmaxf(s, dpp_mov<0xB1>(s));
  if constexpr (W >= 4) s = fmaxf(s, dpp_mov<0x4E>(s));
  if constexpr (W >= 8) s = fmaxf(s, dpp_mov<0x141>(s));
  if constexpr (W >= 16) s = fmaxf(s, dpp_mov<0x140>(s));
  if constexpr (W >= 32) s = fmaxf(s, __shfl_xor(s, 16, 64));
  if constexpr (W >= 64) s = fmaxf(s, __shfl_xor(s, 32, 64));
  return s;
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) { return lane_group_max<64>(v); }

// Remaps a linear workgroup id so that consecutive logical tiles land on the same
// XCD. The dispatcher hands workgroup i to XCD i % 8; logical tile t is executed by
// the workgroup whose id places it on XCD t / ceil(n/8). Valid for any n.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int per = (n + 7) / 8;      // logical tiles per XCD (last XCDs may get fewer)
  const int full = n % 8 == 0 ? 8 : n % 8;  // XCDs that receive `per` workgroups
  const int xcd = bid % 8, slot = bid / 8;
  // XCDs [0, full) hold `per` workgroups, the rest hold per-1.
  return xcd < full ? xcd * per + slot : full * per + (xcd - full) * (per - 1) + slot;
}

}  // namespace mls
