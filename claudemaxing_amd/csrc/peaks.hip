// On-box probes of the two roofline denominators (measurement only; no counterpart in the
// reference): the HBM bandwidth a streaming kernel attains on this board, and the fp16
// matrix-core rate of v_mfma_f32_32x32x16_f16 with register operands. bench.py reports both
// beside the published peaks (8 TB/s, 2.5 PFLOP/s), which the board reaches only at its top
// clock and power.
//
// HBM: one pass over 16-byte words, each workgroup a contiguous span of PER_LANE x 4 KiB
// (PER_LANE loads per lane, plain or nontemporal, all issued before any is used), either
// XOR-reduced (read only; a word is written only if the reduction hits a sentinel, so the loads
// stay live) or stored to a second buffer with nontemporal stores (copy). Few words per lane and
// many workgroups keep reads and writes interleaved; many words per lane put more loads in
// flight; bench.py takes the best.
//
// MFMA: every wavefront keeps CHAINS independent 32 x 32 accumulators and issues 2 x CHAINS
// MFMAs per iteration whose operands alternate between four A and four B fragments of real fp16
// data (the matrix cores draw more power on changing, non-zero operands, which sets the clock);
// the sums are written only if they hit a sentinel. Fewer chains leave more wavefronts per SIMD
// (registers), more chains more independent MFMAs per wavefront; bench.py takes the best.
//
// Launch floor: a kernel whose workgroups do nothing, launched through the same C ABI as the
// library's kernels, so that a kernel trace gives the device time any launch of that grid costs
// on this board (the floor under the small row kernels of a training step).
#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kMfmaBlocks = 2048;
constexpr int64_t kMfmaFlops = 2 * 32 * 32 * 16;

template <int PER_LANE, bool NT_LOAD>
__global__ __launch_bounds__(kThreads) void hbm_stream(const u32x4* __restrict__ src,
                                                       u32x4* __restrict__ dst, int64_t n16,
                                                       uint32_t* __restrict__ sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * PER_LANE + threadIdx.x;
  u32x4 v[PER_LANE];
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int64_t i = base + j * kThreads;
    if (i < n16) {
      v[j] = NT_LOAD ? __builtin_nontemporal_load(src + i) : src[i];
    } else {
      v[j] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (dst) {
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
      const int64_t i = base + j * kThreads;
      if (i < n16) __builtin_nontemporal_store(v[j], dst + i);
    }
    return;
  }
  u32x4 acc = v[0];
#pragma unroll
  for (int j = 1; j < PER_LANE; ++j) acc ^= v[j];
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) sink[0] = r;
}

template <int CHAINS>
__global__ __launch_bounds__(kThreads) void mfma_rate(const half8* __restrict__ operands,
                                                      int iters, float* __restrict__ sink) {
  const int lane = threadIdx.x % cm::kWave;
  half8 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = operands[j * cm::kWave + lane];
    b[j] = operands[(4 + j) * cm::kWave + lane];
  }
  floatx16 acc[CHAINS];
#pragma unroll
  for (int j = 0; j < CHAINS; ++j) acc[j] = floatx16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < CHAINS; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j & 3], b[j & 3], acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < CHAINS; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(j + 1) & 3], b[(j + 2) & 3], acc[j], 0,
                                                      0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < CHAINS; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  if (s == 1234567.0f) sink[0] = s;
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" int cm_probe_launch(int blocks, int threads, void* stream) {
  CM_CHECK_ARG(blocks > 0 && threads > 0 && threads <= 1024 && threads % cm::kWave == 0);
  hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(threads), 0,
                     static_cast<hipStream_t>(stream));
  return cm::launch_status();
}

extern "C" int cm_probe_hbm(const void* src, void* dst, int64_t bytes, int per_lane,
                            int nt_loads, uint32_t* sink, void* stream) {
  CM_CHECK_ARG(src && sink && bytes > 0 && bytes % 16 == 0);
  CM_CHECK_ARG(cm::aligned(src, 16) && (!dst || cm::aligned(dst, 16)));
  CM_CHECK_ARG(per_lane == 1 || per_lane == 4 || per_lane == 16);
  const int64_t n16 = bytes / 16;
  const int64_t per_block = int64_t{kThreads} * per_lane;
  const int64_t blocks = (n16 + per_block - 1) / per_block;
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks));
  const u32x4* in = static_cast<const u32x4*>(src);
  u32x4* out = static_cast<u32x4*>(dst);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, s, in, out, n16, sink);
  };
  if (per_lane == 1) {
    nt_loads ? go(hbm_stream<1, true>) : go(hbm_stream<1, false>);
  } else if (per_lane == 4) {
    nt_loads ? go(hbm_stream<4, true>) : go(hbm_stream<4, false>);
  } else {
    nt_loads ? go(hbm_stream<16, true>) : go(hbm_stream<16, false>);
  }
  return cm::launch_status();
}

extern "C" int64_t cm_probe_mfma_f16_flops(int iters, int chains) {
  if (iters <= 0 || (chains != 2 && chains != 4 && chains != 8)) return 0;
  return int64_t{kMfmaBlocks} * (kThreads / cm::kWave) * iters * 2 * chains * kMfmaFlops;
}

extern "C" int cm_probe_mfma_f16(const void* operands, int iters, int chains, float* sink,
                                 void* stream) {
  CM_CHECK_ARG(operands && sink && iters > 0 && cm::aligned(operands, 16));
  CM_CHECK_ARG(chains == 2 || chains == 4 || chains == 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half8* ops = static_cast<const half8*>(operands);
  if (chains == 2) {
    hipLaunchKernelGGL(mfma_rate<2>, dim3(kMfmaBlocks), dim3(kThreads), 0, s, ops, iters, sink);
  } else if (chains == 4) {
    hipLaunchKernelGGL(mfma_rate<4>, dim3(kMfmaBlocks), dim3(kThreads), 0, s, ops, iters, sink);
  } else {
    hipLaunchKernelGGL(mfma_rate<8>, dim3(kMfmaBlocks), dim3(kThreads), 0, s, ops, iters, sink);
  }
  return cm::launch_status();
}
