// LoRA dropout mask bit-pack / unpack (gfx950), bit-exact.
//
// Reproduces solution/lora.py:30-42 (lora_dropout_pack_kernel) and 45-57
// (lora_dropout_unpack_kernel). Element i of the dropout mask is bit (i % 8) of byte i / 8,
// least significant bit first. pack writes lora_A's input fp16(keep ? x * scale : 0) and the
// bits; unpack rebuilds that input from the fp16 copy of x and returns the input gradient
// keep ? g * scale : 0 in the requested dtype.
//
// A lane handles one mask byte = 8 contiguous elements: x in one 16/32-byte access, the 8 keep
// bytes as one 8-byte access, the fp16 output as one 16-byte store, the bits as one byte store
// (a wavefront stores 64 contiguous bytes). HBM-bound: pack 7.125 B/element for fp32 x,
// unpack 10.125 B/element for an fp32 gradient.
#include "vec.h"

namespace {

#pragma clang fp contract(off)

constexpr int kThreads = 256;
constexpr int kUnits = 2;

template <typename XT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void lora_pack_kernel(const XT* __restrict__ x,
                                                             const uint8_t* __restrict__ keep,
                                                             _Float16* __restrict__ xd,
                                                             uint8_t* __restrict__ bits,
                                                             int64_t n_bytes, float scale) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnits) + threadIdx.x;
#pragma unroll
  for (int j = 0; j < kUnits; ++j) {
    const int64_t b = base + j * kThreads;
    if (b >= n_bytes) return;
    uint32_t k0, k1;
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
    float v[8], o[8];
    cm::Vec8<XT, ALIGNED>::load(x + 8 * b, v);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? k0 : k1) >> (8 * (i & 3))) & 0xffu;
      const bool kept = byte != 0;
      packed |= static_cast<uint32_t>(kept) << i;
      o[i] = kept ? v[i] * scale : 0.0f;
    }
    cm::Vec8<_Float16, ALIGNED>::store(xd + 8 * b, o);
    bits[b] = static_cast<uint8_t>(packed);
  }
}

template <typename DXT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void lora_unpack_kernel(
    const _Float16* __restrict__ x16, const uint8_t* __restrict__ bits,
    const _Float16* __restrict__ g16, _Float16* __restrict__ xd, DXT* __restrict__ dx,
    int64_t n_bytes, float scale) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnits) + threadIdx.x;
#pragma unroll
  for (int j = 0; j < kUnits; ++j) {
    const int64_t b = base + j * kThreads;
    if (b >= n_bytes) return;
    const uint32_t m = bits[b];
    float xv[8], gv[8], xo[8], go[8];
    cm::Vec8<_Float16, ALIGNED>::load(x16 + 8 * b, xv);
    cm::Vec8<_Float16, ALIGNED>::load(g16 + 8 * b, gv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool kept = (m >> i) & 1u;
      xo[i] = kept ? xv[i] * scale : 0.0f;
      go[i] = kept ? gv[i] * scale : 0.0f;
    }
    cm::Vec8<_Float16, ALIGNED>::store(xd + 8 * b, xo);
    cm::Vec8<DXT, ALIGNED>::store(dx + 8 * b, go);
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
  const int64_t n_bytes = n / 8;
  const int64_t blocks = grid_for(n_bytes);
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool al = cm::aligned(x16, 16) && cm::aligned(g16, 16) && cm::aligned(xd16, 16) &&
                  cm::aligned(dx, 16);
  CM_FLOAT_SWITCH(dx_dtype, DXT, {
    if (al)
      hipLaunchKernelGGL((lora_unpack_kernel<DXT, true>), dim3(blocks), dim3(kThreads), 0, s,
                         static_cast<const _Float16*>(x16), bits,
                         static_cast<const _Float16*>(g16), static_cast<_Float16*>(xd16),
                         static_cast<DXT*>(dx), n_bytes, scale);
    else
      hipLaunchKernelGGL((lora_unpack_kernel<DXT, false>), dim3(blocks), dim3(kThreads), 0, s,
                         static_cast<const _Float16*>(x16), bits,
                         static_cast<const _Float16*>(g16), static_cast<_Float16*>(xd16),
                         static_cast<DXT*>(dx), n_bytes, scale);
  });
  return cm::launch_status();
}
