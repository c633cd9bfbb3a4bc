// 8-element vector loads/stores with conversion to/from fp32, for the elementwise kernels.
// A vector of 8 elements is 16 B for 16-bit types and 32 B for fp32; the caller guarantees
// 16-byte alignment of every 8-element group (ALIGNED = true) or uses the element-wise form.
#pragma once

#include "common.h"

namespace cm {

template <typename T, bool ALIGNED>
struct Vec8 {
  // Load elements [0, cnt) of p (cnt <= 8); the rest are 0.
  static __device__ __forceinline__ void load(const T* p, float (&v)[8], int cnt = 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = i < cnt ? to_f32(p[i]) : 0.0f;
  }
  static __device__ __forceinline__ void store(T* p, const float (&v)[8], int cnt = 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < cnt) p[i] = from_f32<T>(v[i]);
  }
};

template <>
struct Vec8<_Float16, true> {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ void load(const _Float16* p, float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      const h8 h = *reinterpret_cast<const h8*>(p);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(h[i]);
    } else {
      Vec8<_Float16, false>::load(p, v, cnt);
    }
  }
  static __device__ __forceinline__ void store(_Float16* p, const float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      h8 h;
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = from_f32<_Float16>(v[i]);
      *reinterpret_cast<h8*>(p) = h;
    } else {
      Vec8<_Float16, false>::store(p, v, cnt);
    }
  }
};

template <>
struct Vec8<bf16_t, true> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      const uint4 w = *reinterpret_cast<const uint4*>(p);
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      }
    } else {
      Vec8<bf16_t, false>::load(p, v, cnt);
    }
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      uint32_t u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        u[i] = static_cast<uint32_t>(from_f32<bf16_t>(v[2 * i]).bits) |
               (static_cast<uint32_t>(from_f32<bf16_t>(v[2 * i + 1]).bits) << 16);
      *reinterpret_cast<uint4*>(p) = make_uint4(u[0], u[1], u[2], u[3]);
    } else {
      Vec8<bf16_t, false>::store(p, v, cnt);
    }
  }
};

template <>
struct Vec8<float, true> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      const float4 a = reinterpret_cast<const float4*>(p)[0];
      const float4 b = reinterpret_cast<const float4*>(p)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      Vec8<float, false>::load(p, v, cnt);
    }
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      Vec8<float, false>::store(p, v, cnt);
    }
  }
};

}  // namespace cm
