// Shared helpers for the gfx950 kernels: status reporting, element types,
// 16-byte vector loads and wave64 lane reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <type_traits>

#include "../../include/pagelora.h"

namespace pl {

// A pointer rebuilt from integer bits (kernel arguments held in SGPRs by an
// empty asm statement), marked as global memory first: a pointer made
// straight from an integer compiles to flat accesses, which wait on both the
// vector and the scalar memory counters.
template <typename P>
__device__ __forceinline__ P gptr(uint64_t u) {
  using E = typename std::remove_pointer<P>::type;
  return (P)(__attribute__((address_space(1))) E*)u;
}

// ---------------------------------------------------------------- errors ---
// The message buffer is per host thread, so concurrent callers on different
// threads do not clobber each other's diagnostics.
inline char* error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

inline int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return status;
}

inline int ok() {
  error_buffer()[0] = 0;
  return PL_OK;
}

#define PL_HIP_CHECK(expr)                                                  \
  do {                                                                      \
    hipError_t _e = (expr);                                                 \
    if (_e != hipSuccess)                                                   \
      return ::pl::fail(PL_ERR_HIP, "%s failed: %s", #expr,                 \
                        hipGetErrorString(_e));                             \
  } while (0)

// After a kernel launch: report launch-configuration errors synchronously.
#define PL_LAUNCH_CHECK(name)                                               \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess)                                                   \
      return ::pl::fail(PL_ERR_HIP, "launch of %s failed: %s", name,        \
                        hipGetErrorString(_e));                             \
  } while (0)

// --------------------------------------------------------- element types ---
// Storage types.  bf16 is kept as raw 16-bit words; every conversion below
// rounds to nearest even.
struct bf16_t { uint16_t x; };
typedef _Float16 f16_t;

template <typename T> struct ElemBytes;
template <> struct ElemBytes<float> { static constexpr int value = 4; };
template <> struct ElemBytes<f16_t> { static constexpr int value = 2; };
template <> struct ElemBytes<bf16_t> { static constexpr int value = 2; };

__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round to nearest even with the hardware conversion (v_cvt_pk_bf16_f32, one
// instruction per pair): the bits of (u + 0x7fff + ((u >> 16) & 1)) >> 16
// for every non-NaN float u; a NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return (uint16_t)f32x2_to_bf16x2_bits(f, f);
}

__device__ __forceinline__ float h_lo(uint32_t w) {
  half2_t h = __builtin_bit_cast(half2_t, w);
  return (float)h.x;
}
__device__ __forceinline__ float h_hi(uint32_t w) {
  half2_t h = __builtin_bit_cast(half2_t, w);
  return (float)h.y;
}

// Unpack two packed 16-bit values of type T into floats.
template <typename T> __device__ __forceinline__ void unpack2(uint32_t w, float& a, float& b);
template <> __device__ __forceinline__ void unpack2<bf16_t>(uint32_t w, float& a, float& b) {
  a = bf16_lo(w);
  b = bf16_hi(w);
}
template <> __device__ __forceinline__ void unpack2<f16_t>(uint32_t w, float& a, float& b) {
  a = h_lo(w);
  b = h_hi(w);
}

// fp32 dot of two packed pairs plus c: v_dot2_f32_{f16,bf16}.
template <typename T> __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);
template <> __device__ __forceinline__ float dot2<f16_t>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                __builtin_bit_cast(half2_t, b), c, false);
}
template <> __device__ __forceinline__ float dot2<bf16_t>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Store one float as T.
template <typename T> __device__ __forceinline__ T from_float(float f);
template <> __device__ __forceinline__ float from_float<float>(float f) { return f; }
template <> __device__ __forceinline__ f16_t from_float<f16_t>(float f) { return (f16_t)f; }
template <> __device__ __forceinline__ bf16_t from_float<bf16_t>(float f) {
  bf16_t r;
  r.x = f32_to_bf16_bits(f);
  return r;
}
template <typename T> __device__ __forceinline__ float to_float(T v);
template <> __device__ __forceinline__ float to_float<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_float<f16_t>(f16_t v) { return (float)v; }
template <> __device__ __forceinline__ float to_float<bf16_t>(bf16_t v) {
  return __uint_as_float(((uint32_t)v.x) << 16);
}

// Pack two floats into one 32-bit word of two T (16-bit types only).
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
  return f32x2_to_bf16x2_bits(a, b);
}
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) {
  half2_t h;
  h.x = (f16_t)a;
  h.y = (f16_t)b;
  return __builtin_bit_cast(uint32_t, h);
}

// pack2 by the hardware conversion for both types (bf16's pack2 is that
// conversion too).
template <typename T> __device__ __forceinline__ uint32_t pack2_hw(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2_hw<bf16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack2_hw<f16_t>(float a, float b) { return pack2<f16_t>(a, b); }

// ------------------------------------------------------- lane reductions ---
// All-reduce across the 16 lanes of a DPP row with row rotations; every lane
// of the row ends with the full result.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<0x128>(x);  // row_ror:8
  x += dpp_mov<0x124>(x);  // row_ror:4
  x += dpp_mov<0x122>(x);  // row_ror:2
  x += dpp_mov<0x121>(x);  // row_ror:1
  return x;
}
__device__ __forceinline__ float row8_sum(float x) {  // within aligned groups of 8 lanes
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 1);
  return x;
}
__device__ __forceinline__ float row32_sum(float x) {  // within aligned groups of 32 lanes
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  return x;
}

// Wave-wide reductions: DPP within each 16-lane row, then the four row
// results read into scalar registers (no LDS round trips, the same value in
// every lane).
__device__ __forceinline__ float lane_value(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_mov<0x128>(x));  // row_ror:8
  x = fmaxf(x, dpp_mov<0x124>(x));  // row_ror:4
  x = fmaxf(x, dpp_mov<0x122>(x));  // row_ror:2
  x = fmaxf(x, dpp_mov<0x121>(x));  // row_ror:1
  return fmaxf(fmaxf(lane_value(x, 0), lane_value(x, 16)), fmaxf(lane_value(x, 32), lane_value(x, 48)));
}
__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  return (lane_value(x, 0) + lane_value(x, 16)) + (lane_value(x, 32) + lane_value(x, 48));
}

// All-reduce over aligned groups of 2^lg lanes (0 <= lg <= 6, wave
// uniform) with DPP and lane reads, no LDS traffic; every lane of a group
// gets the group's sum (lanes of one group may associate the terms in
// different orders, each lane always the same way).
__device__ __forceinline__ float group_sum(float x, int lg) {
  if (lg >= 4) {
    x = row16_sum(x);
    if (lg == 4) return x;
    const float r0 = lane_value(x, 0), r1 = lane_value(x, 16), r2 = lane_value(x, 32), r3 = lane_value(x, 48);
    if (lg == 6) return (r0 + r1) + (r2 + r3);
    return (threadIdx.x & 32) ? r2 + r3 : r0 + r1;
  }
  if (lg == 3) {
    x += dpp_mov<0x141>(x);  // row_half_mirror: lane i of each 8 with lane 7 - i
    x += dpp_mov<0x1b>(x);   // quad_perm [3,2,1,0]
    return x + dpp_mov<0xb1>(x);  // quad_perm [1,0,3,2]
  }
  if (lg >= 1) x += dpp_mov<0xb1>(x);  // quad_perm [1,0,3,2]
  if (lg == 2) x += dpp_mov<0x4e>(x);  // quad_perm [2,3,0,1]
  return x;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// exp2 on the hardware transcendental unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

inline int dtype_bytes(int dtype) {
  return dtype == PL_DTYPE_F32 ? 4 : 2;
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// k-slices of the LoRA shrink: at least 512 elements per slice, and fewer
// slices as tokens grow so the expand's fold stays short.  Shared by the
// shrink and by every consumer of its partials.
inline int lora_ksplit(int tokens, int in_features) {
  int by_k = in_features / 512;
  int by_t = 256 / (tokens > 0 ? tokens : 1);
  int k = by_k < by_t ? by_k : by_t;
  return k < 1 ? 1 : (k > 64 ? 64 : k);
}

}  // namespace pl
