// Online softmax statistics of a set of logits: running maximum M, S = sum e^{z-M},
// D = sum e^{z-M} z and the first index of the maximum. Used by the cross-entropy kernels;
// lse = M + ln S, entropy = lse - D / S.
#pragma once

#include "common.h"

namespace cm {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// e^x via v_exp_f32 (2^x) and ln x via v_log_f32 (log2 x); about 1 ulp of the exact values
// away for the arguments used here.
__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float log_f(float x) { return __builtin_amdgcn_logf(x) * kLn2; }
// ln(1 + x) for x >= 0 without the rounding of 1 + x near 0: the alternating Taylor series
// through x^6 for x < 1/32 (the first omitted term is below 2^-37 of the result), log_f(1 + x)
// beyond.
__device__ __forceinline__ float log1p_f(float x) {
  if (x < 0.03125f)
    return x * (1.0f - x * (0.5f - x * (1.0f / 3 - x * (0.25f - x * (0.2f - x * (1.0f / 6))))));
  return log_f(1.0f + x);
}

struct SoftmaxState {
  float max;
  float sum;
  float dot;
  int64_t best;

  static __device__ __forceinline__ SoftmaxState empty() {
    return SoftmaxState{-__builtin_huge_valf(), 0.0f, 0.0f, int64_t{0x7fffffffffffffff}};
  }

  // Add logit z at column c; columns must arrive in increasing order per state.
  __device__ __forceinline__ void push(float z, int64_t c) {
    if (z > max) {
      const float r = exp_f(max - z);  // 0 while the state is empty
      sum *= r;
      dot *= r;
      max = z;
      best = c;
    }
    const float e = exp_f(z - max);
    sum += e;
    dot += e * z;
  }

  __device__ __forceinline__ void merge(const SoftmaxState& o) {
    if (o.max == -__builtin_huge_valf()) return;
    if (max == -__builtin_huge_valf()) {
      *this = o;
      return;
    }
    const float m = fmaxf(max, o.max);
    const float ra = exp_f(max - m), rb = exp_f(o.max - m);
    sum = sum * ra + o.sum * rb;
    dot = dot * ra + o.dot * rb;
    if (o.max > max || (o.max == max && o.best < best)) best = o.best;
    max = m;
  }

  __device__ __forceinline__ float lse() const { return max + log_f(sum); }
};

__device__ __forceinline__ SoftmaxState shfl_xor_state(const SoftmaxState& s, int off) {
  SoftmaxState o;
  o.max = __shfl_xor(s.max, off, kWave);
  o.sum = __shfl_xor(s.sum, off, kWave);
  o.dot = __shfl_xor(s.dot, off, kWave);
  o.best = __shfl_xor(s.best, off, kWave);
  return o;
}

__device__ __forceinline__ SoftmaxState wave_merge(SoftmaxState s) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s.merge(shfl_xor_state(s, off));
  return s;
}

// Merge the states of all lanes of a THREADS-lane workgroup; every lane gets the result.
template <int THREADS>
__device__ __forceinline__ SoftmaxState block_merge(SoftmaxState s, SoftmaxState* part) {
  s = wave_merge(s);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) part[wave] = s;
  __syncthreads();
  SoftmaxState r = part[0];
#pragma unroll
  for (int i = 1; i < THREADS / kWave; ++i) r.merge(part[i]);
  return r;
}

}  // namespace cm
