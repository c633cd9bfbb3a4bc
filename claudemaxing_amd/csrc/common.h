// Shared device/host helpers of the gfx950 kernel library: element types, conversions with
// round-to-nearest-even, wavefront reductions and the argument/launch checks of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "claudemaxing_amd.h"

namespace cm {

constexpr int kWave = 64;  // CDNA wavefront width

// ------------------------------------------------------------------------------------------
// Element types. fp16 is clang's _Float16 (v_cvt_f16_f32 rounds to nearest even); bf16 is kept
// as raw bits and converted by hand with round-to-nearest-even.
struct bf16_t {
  uint16_t bits;
};

template <typename T>
struct Conv;

template <>
struct Conv<float> {
  static __device__ __forceinline__ float load(float v) { return v; }
  static __device__ __forceinline__ float store(float v) { return v; }
};

// Pins an fp32 value in a register as it is. The compiler would otherwise fold an fp32
// multiply followed by the conversion to fp16 into one mixed-precision instruction
// (v_fma_mix*_f16) that rounds the exact product once; the reference rounds twice (to fp32,
// then to fp16), and the two differ in the last fp16 bit for a few products in 10^5.
__device__ __forceinline__ float materialize(float v) {
  asm("" : "+v"(v));
  return v;
}

template <>
struct Conv<_Float16> {
  static __device__ __forceinline__ float load(_Float16 v) { return static_cast<float>(v); }
  static __device__ __forceinline__ _Float16 store(float v) {
    return static_cast<_Float16>(materialize(v));
  }
};

template <>
struct Conv<bf16_t> {
  static __device__ __forceinline__ float load(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
  }
  static __device__ __forceinline__ bf16_t store(float v) {
    uint32_t u = __float_as_uint(v);
    bf16_t r;
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      r.bits = static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN, sign kept
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
      r.bits = static_cast<uint16_t>(u >> 16);
    }
    return r;
  }
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return Conv<T>::load(v);
}
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return Conv<T>::store(v);
}
// Round an fp32 value to T and back (the reference's `.to(dtype).to(float32)`).
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  return Conv<T>::load(Conv<T>::store(v));
}

// ------------------------------------------------------------------------------------------
// Wavefront reductions (64 lanes) through cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// ------------------------------------------------------------------------------------------
// Host-side helpers.
inline bool is_float_dtype(int dt) { return dt == CM_F32 || dt == CM_F16 || dt == CM_BF16; }

inline int dtype_size(int dt) {
  switch (dt) {
    case CM_F32: return 4;
    case CM_F16: return 2;
    case CM_BF16: return 2;
    case CM_U8: return 1;
    case CM_I32: return 4;
    case CM_I64: return 8;
    default: return 0;
  }
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int launch_status() { return static_cast<int>(hipGetLastError()); }

}  // namespace cm

#define CM_CHECK_ARG(cond)                                     \
  do {                                                          \
    if (!(cond)) return static_cast<int>(hipErrorInvalidValue); \
  } while (0)

// Dispatch a float dtype code to a type alias, for templated kernels.
#define CM_FLOAT_SWITCH(dt, T, ...)         \
  switch (dt) {                             \
    case CM_F32: {                          \
      using T = float;                      \
      __VA_ARGS__;                          \
    } break;                                \
    case CM_F16: {                          \
      using T = _Float16;                   \
      __VA_ARGS__;                          \
    } break;                                \
    case CM_BF16: {                         \
      using T = cm::bf16_t;                 \
      __VA_ARGS__;                          \
    } break;                                \
    default:                                \
      return static_cast<int>(hipErrorInvalidValue); \
  }
