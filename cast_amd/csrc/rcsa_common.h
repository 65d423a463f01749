// Shared device helpers for the gfx950 RCSA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rcsa.h"

namespace rcsa {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short u16;

constexpr int kWave = 64;
constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

// bf16 <-> fp32 by bit manipulation (round to nearest even on the way down).
__device__ __forceinline__ float bf16_to_f32(u16 h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ u16 f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) {  // inf / nan: keep, force quiet nan
    return static_cast<u16>((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<u16>(u >> 16);
}
// Two floats -> packed bf16x2 (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16(a)) |
         (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// Loads of 8 consecutive elements (16 bytes of bf16, 32 bytes of fp32) as fp32.
template <typename T>
struct Vec8;
template <>
struct Vec8<u16> {
  static __device__ __forceinline__ void load(const u16* p, float* out) {
    uint4 r = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float* out) {
    float4 a = *reinterpret_cast<const float4*>(p);
    float4 b = *reinterpret_cast<const float4*>(p + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
};

// Round-to-nearest-even float -> int8 in [-127, 127].
__device__ __forceinline__ int quant_i8(float x, float inv_scale) {
  float r = __builtin_rintf(x * inv_scale);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<int>(r);
}

// Wavefront reductions (64 lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RCSA_OK : RCSA_ERR_LAUNCH;
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace rcsa
