// 8-element vector loads/stores with conversion to/from fp32, for the elementwise kernels.
// A vector of 8 elements is 16 B for 16-bit types and 32 B for fp32; the caller guarantees
// 16-byte alignment of every 8-element group (ALIGNED = true) or uses the element-wise form.
#pragma once

#include "common.h"

// Streaming hints for the aligned 16-byte accesses. Stores are nontemporal (streaming): measured
// on MI355X with cold caches, they speed up every elementwise kernel here (SwiGLU forward
// 21.0 -> 18.6 us, RMSNorm backward 8.0 -> 6.5 us, LoRA unpack 5.7 -> 4.9 us). Loads are
// nontemporal only where a kernel asks (Vec8's STREAM): that helps kernels that read each input
// once (SwiGLU backward 35.8 -> 30.9 us) and slows RMSNorm, which reads its rows twice.
namespace cm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes at p (16-byte aligned), as any 16-byte type V; STREAM = a nontemporal load.
template <typename V, bool STREAM = false>
__device__ __forceinline__ V load16(const void* p) {
  static_assert(sizeof(V) == 16, "16-byte accesses only");
  if constexpr (STREAM) {
    return __builtin_bit_cast(V, __builtin_nontemporal_load(static_cast<const u32x4*>(p)));
  } else {
    return __builtin_bit_cast(V, *static_cast<const u32x4*>(p));
  }
}

// 16 bytes to p (16-byte aligned), nontemporal.
template <typename V>
__device__ __forceinline__ void store16(void* p, V v) {
  static_assert(sizeof(V) == 16, "16-byte accesses only");
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), static_cast<u32x4*>(p));
}

// Eight elements of T at a time, converted to and from fp32. ALIGNED: every 8-element group is
// 16-byte aligned (16-byte accesses); STREAM: its loads are nontemporal.
template <typename T, bool ALIGNED, bool STREAM = false>
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

template <bool STREAM>
struct Vec8<_Float16, true, STREAM> {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ void load(const _Float16* p, float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      const h8 h = load16<h8, STREAM>(p);
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
      store16(p, h);
    } else {
      Vec8<_Float16, false>::store(p, v, cnt);
    }
  }
};

template <bool STREAM>
struct Vec8<bf16_t, true, STREAM> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      const uint4 w = load16<uint4, STREAM>(p);
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
      store16(p, make_uint4(u[0], u[1], u[2], u[3]));
    } else {
      Vec8<bf16_t, false>::store(p, v, cnt);
    }
  }
};

template <bool STREAM>
struct Vec8<float, true, STREAM> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      const float4 a = load16<float4, STREAM>(p);
      const float4 b = load16<float4, STREAM>(p + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      Vec8<float, false>::load(p, v, cnt);
    }
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8], int cnt = 8) {
    if (cnt == 8) {
      store16(p, make_float4(v[0], v[1], v[2], v[3]));
      store16(p + 4, make_float4(v[4], v[5], v[6], v[7]));
    } else {
      Vec8<float, false>::store(p, v, cnt);
    }
  }
};

}  // namespace cm
