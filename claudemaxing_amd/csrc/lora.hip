// LoRA dropout mask bit-pack / unpack (gfx950), bit-exact.
//
// Reproduces solution/lora.py:30-42 (lora_dropout_pack_kernel) and 45-57
// (lora_dropout_unpack_kernel). Element i of the dropout mask is bit (i % 8) of byte i / 8,
// least significant bit first. pack writes lora_A's input fp16(keep ? x * scale : 0) and the
// bits; unpack rebuilds that input from the fp16 copy of x and returns the input gradient
// keep ? g * scale : 0 in the requested dtype.
//
// pack: a lane handles one mask byte = 8 contiguous elements: x in one 16/32-byte access, the 8
// keep bytes as one 8-byte access, the fp16 output as one 16-byte store, the bits as one byte
// store (a wavefront stores 64 contiguous bytes). unpack: a lane handles quads of 4 elements.
// HBM-bound: pack 7.125 B/element for fp32 x, unpack 10.125 B/element for an fp32 gradient.
#include <type_traits>

#include "vec.h"

namespace {

#pragma clang fp contract(off)

constexpr int kThreads = 256;
constexpr int kUnits = 2;

// One mask byte: 8 elements of x, their 8 keep bytes -> 8 fp16 outputs and the packed byte.
template <typename XT, bool ALIGNED>
struct PackUnit {
  float v[8];
  uint32_t k0, k1;

  __device__ __forceinline__ void load(const XT* x, const uint8_t* keep, int64_t b) {
    if (ALIGNED) {
      const uint2 kk = *reinterpret_cast<const uint2*>(keep + 8 * b);
      k0 = kk.x;
      k1 = kk.y;
    } else {
      k0 = k1 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        k0 |= static_cast<uint32_t>(keep[8 * b + i]) << (8 * i);
        k1 |= static_cast<uint32_t>(keep[8 * b + 4 + i]) << (8 * i);
      }
    }
    cm::Vec8<XT, ALIGNED>::load(x + 8 * b, v);
  }
  __device__ __forceinline__ void store(_Float16* xd, uint8_t* bits, int64_t b, float scale) const {
    float o[8];
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool kept = (((i < 4 ? k0 : k1) >> (8 * (i & 3))) & 0xffu) != 0;
      packed |= static_cast<uint32_t>(kept) << i;
      o[i] = kept ? v[i] * scale : 0.0f;
    }
    cm::Vec8<_Float16, ALIGNED>::store(xd + 8 * b, o);
    bits[b] = static_cast<uint8_t>(packed);
  }
};

// A workgroup covers kUnits * kThreads mask bytes; when all of them exist every load is issued
// before the first store (one memory round trip), otherwise unit by unit with a bound test.
template <typename XT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void lora_pack_kernel(const XT* __restrict__ x,
                                                             const uint8_t* __restrict__ keep,
                                                             _Float16* __restrict__ xd,
                                                             uint8_t* __restrict__ bits,
                                                             int64_t n_bytes, float scale) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnits) + threadIdx.x;
  PackUnit<XT, ALIGNED> u[kUnits];
  if (base + (kUnits - 1) * kThreads < n_bytes) {
#pragma unroll
    for (int j = 0; j < kUnits; ++j) u[j].load(x, keep, base + j * kThreads);
#pragma unroll
    for (int j = 0; j < kUnits; ++j) u[j].store(xd, bits, base + j * kThreads, scale);
    return;
  }
  for (int j = 0; j < kUnits && base + j * kThreads < n_bytes; ++j) {
    u[0].load(x, keep, base + j * kThreads);
    u[0].store(xd, bits, base + j * kThreads, scale);
  }
}

// The backward works on quads: 4 elements, half a mask byte. Every access of a wavefront is
// then contiguous: 512 B per fp16 load or store and 1 KiB per fp32 gradient store, where
// 8-element lanes store an fp32 gradient as two 16-byte halves 32 B apart (the quad form runs
// at 87 us instead of 100 us over [32768, 1536] on MI355X).
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <bool ALIGNED>
__device__ __forceinline__ void load_quad(const _Float16* p, float (&v)[4]) {
  if (ALIGNED) {
    const h4 h = *reinterpret_cast<const h4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = static_cast<float>(h[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = static_cast<float>(p[i]);
  }
}

template <typename T, bool ALIGNED>
__device__ __forceinline__ void store_quad(T* p, const float (&v)[4]) {
  if constexpr (!ALIGNED) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = cm::from_f32<T>(v[i]);
  } else if constexpr (std::is_same<T, float>::value) {
    cm::store16(p, make_float4(v[0], v[1], v[2], v[3]));
  } else {
    uint32_t u[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      u[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, cm::from_f32<T>(v[2 * i]))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, cm::from_f32<T>(v[2 * i + 1])))
              << 16);
    const u32x2 w = {u[0], u[1]};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(p));
  }
}

template <typename DXT, bool ALIGNED>
struct UnpackQuad {
  float xv[4], gv[4];
  uint32_t m;  // the quad's 4 mask bits in bits 0-3

  __device__ __forceinline__ void load(const _Float16* x16, const uint8_t* bits,
                                       const _Float16* g16, int64_t q) {
    m = static_cast<uint32_t>(bits[q >> 1]) >> (4 * (q & 1));
    load_quad<ALIGNED>(x16 + 4 * q, xv);
    load_quad<ALIGNED>(g16 + 4 * q, gv);
  }
  __device__ __forceinline__ void store(_Float16* xd, DXT* dx, int64_t q, float scale) const {
    float xo[4], go[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool kept = (m >> i) & 1u;
      xo[i] = kept ? xv[i] * scale : 0.0f;
      go[i] = kept ? gv[i] * scale : 0.0f;
    }
    store_quad<_Float16, ALIGNED>(xd + 4 * q, xo);
    store_quad<DXT, ALIGNED>(dx + 4 * q, go);
  }
};

constexpr int kQuadUnits = 4;

// A workgroup covers kQuadUnits * kThreads quads; when all of them exist every load is issued
// before the first store, otherwise quad by quad with a bound test.
template <typename DXT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void lora_unpack_kernel(
    const _Float16* __restrict__ x16, const uint8_t* __restrict__ bits,
    const _Float16* __restrict__ g16, _Float16* __restrict__ xd, DXT* __restrict__ dx,
    int64_t n_quads, float scale) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kQuadUnits) + threadIdx.x;
  UnpackQuad<DXT, ALIGNED> u[kQuadUnits];
  if (base + (kQuadUnits - 1) * kThreads < n_quads) {
#pragma unroll
    for (int j = 0; j < kQuadUnits; ++j) u[j].load(x16, bits, g16, base + j * kThreads);
#pragma unroll
    for (int j = 0; j < kQuadUnits; ++j) u[j].store(xd, dx, base + j * kThreads, scale);
    return;
  }
  for (int j = 0; j < kQuadUnits && base + j * kThreads < n_quads; ++j) {
    u[0].load(x16, bits, g16, base + j * kThreads);
    u[0].store(xd, dx, base + j * kThreads, scale);
  }
}

int64_t grid_for(int64_t n_bytes) {
  const int64_t per_block = int64_t{kThreads} * kUnits;
  return (n_bytes + per_block - 1) / per_block;
}

}  // namespace

extern "C" int cm_lora_pack(const void* x, int x_dtype, const uint8_t* keep, void* xd16,
                            uint8_t* bits, int64_t n, float scale, void* stream) {
  CM_CHECK_ARG(n >= 0 && n % 8 == 0);
  if (n == 0) return 0;
  CM_CHECK_ARG(x && keep && xd16 && bits);
  const int64_t n_bytes = n / 8;
  const int64_t blocks = grid_for(n_bytes);
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool al = cm::aligned(x, 16) && cm::aligned(keep, 8) && cm::aligned(xd16, 16);
  CM_FLOAT_SWITCH(x_dtype, XT, {
    if (al)
      hipLaunchKernelGGL((lora_pack_kernel<XT, true>), dim3(blocks), dim3(kThreads), 0, s,
                         static_cast<const XT*>(x), keep, static_cast<_Float16*>(xd16), bits,
                         n_bytes, scale);
    else
      hipLaunchKernelGGL((lora_pack_kernel<XT, false>), dim3(blocks), dim3(kThreads), 0, s,
                         static_cast<const XT*>(x), keep, static_cast<_Float16*>(xd16), bits,
                         n_bytes, scale);
  });
  return cm::launch_status();
}

extern "C" int cm_lora_unpack(const void* x16, const uint8_t* bits, const void* g16, void* xd16,
                              void* dx, int dx_dtype, int64_t n, float scale, void* stream) {
  CM_CHECK_ARG(n >= 0 && n % 8 == 0);
  if (n == 0) return 0;
  CM_CHECK_ARG(x16 && bits && g16 && xd16 && dx);
  const int64_t n_quads = n / 4;
  const int64_t per_block = int64_t{kThreads} * kQuadUnits;
  const int64_t blocks = (n_quads + per_block - 1) / per_block;
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool al16 = cm::aligned(x16, 8) && cm::aligned(g16, 8) && cm::aligned(xd16, 8);
  CM_FLOAT_SWITCH(dx_dtype, DXT, {
    if (al16 && cm::aligned(dx, 4 * sizeof(DXT)))
      hipLaunchKernelGGL((lora_unpack_kernel<DXT, true>), dim3(blocks), dim3(kThreads), 0, s,
                         static_cast<const _Float16*>(x16), bits,
                         static_cast<const _Float16*>(g16), static_cast<_Float16*>(xd16),
                         static_cast<DXT*>(dx), n_quads, scale);
    else
      hipLaunchKernelGGL((lora_unpack_kernel<DXT, false>), dim3(blocks), dim3(kThreads), 0, s,
                         static_cast<const _Float16*>(x16), bits,
                         static_cast<const _Float16*>(g16), static_cast<_Float16*>(xd16),
                         static_cast<DXT*>(dx), n_quads, scale);
  });
  return cm::launch_status();
}
