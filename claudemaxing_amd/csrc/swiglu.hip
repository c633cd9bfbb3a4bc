// SwiGLU of the Qwen2 MLP, silu(gate) * up, forward and recompute-backward (gfx950).
//
// Reproduces solution/swiglu_recompute.py:36-48 (silu_mul_fwd_persistent) and 51-79
// (silu_mul_bwd_recompute): silu(g) = g / (1 + 2^(-g*log2 e)), optionally rounded to the gate
// dtype before it meets `up` (ROUND_SILU), the gradient of the product rounded to the gate
// dtype before it goes back through silu; backward recomputes silu from gate instead of reading
// a saved copy and may write its gradients over gate/up (each element is read before written).
//
// HBM-bound: 6 B/element forward, 10 B/element backward for fp16. A lane handles 8 contiguous
// elements per vector (16-byte fp16 accesses), UNITS vectors per lane, 256 lanes per workgroup;
// consecutive lanes touch consecutive 16-byte vectors so each wavefront access is one
// contiguous 1 KiB span. 2^x is v_exp_f32 and 1/x is v_rcp_f32 (about 1 ulp each; the
// reference's Triton exp2 and division are not correctly rounded either). Every input element
// is read exactly once, so loads and stores are both nontemporal.
#include "vec.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnits = 1;  // 8-element vectors per lane
constexpr float kNegLog2e = -1.4426950408889634f;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// The per-vector arithmetic, shared by the flat and the row-strided kernels.
template <typename GT>
__device__ __forceinline__ void silu_mul8(const float (&g)[8], const float (&u)[8], float (&o)[8],
                                          int round_silu) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float s = g[i] * rcp_fast(1.0f + exp2_fast(g[i] * kNegLog2e));
    if (round_silu) s = cm::round_to<GT>(s);
    o[i] = s * u[i];
  }
}

template <typename GT>
__device__ __forceinline__ void silu_mul_grad8(const float (&d)[8], const float (&g)[8],
                                               const float (&u)[8], float (&dg)[8],
                                               float (&du)[8], int want_dgate, int round_silu) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float sig = rcp_fast(1.0f + exp2_fast(g[i] * kNegLog2e));
    float silu = g[i] * sig;
    if (round_silu) silu = cm::round_to<GT>(silu);
    du[i] = d[i] * silu;
    float dsilu = want_dgate ? d[i] * u[i] : 0.0f;
    if (round_silu) dsilu = cm::round_to<GT>(dsilu);
    dg[i] = dsilu * sig * (1.0f + g[i] * (1.0f - sig));
  }
}

template <typename GT, typename UT, typename OT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_kernel(const GT* __restrict__ gate,
                                                              const UT* __restrict__ up,
                                                              OT* __restrict__ out, int64_t n,
                                                              int round_silu) {
  const int64_t n_vec = (n + 7) / 8;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnits) + threadIdx.x;
#pragma unroll
  for (int j = 0; j < kUnits; ++j) {
    const int64_t vi = base + j * kThreads;
    if (vi >= n_vec) return;
    const int64_t e0 = vi * 8;
    const int cnt = n - e0 >= 8 ? 8 : static_cast<int>(n - e0);
    float g[8], u[8], o[8];
    cm::Vec8<GT, ALIGNED, true>::load(gate + e0, g, cnt);
    cm::Vec8<UT, ALIGNED, true>::load(up + e0, u, cnt);
    silu_mul8<GT>(g, u, o, round_silu);
    cm::Vec8<OT, ALIGNED>::store(out + e0, o, cnt);
  }
}

// dgate may alias gate and dup may alias up: no __restrict__ on those.
template <typename DT, typename GT, typename UT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(const DT* __restrict__ dy,
                                                              const GT* gate, const UT* up,
                                                              GT* dgate, UT* dup, int64_t n,
                                                              int want_dgate, int want_dup,
                                                              int round_silu) {
  const int64_t n_vec = (n + 7) / 8;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnits) + threadIdx.x;
#pragma unroll
  for (int j = 0; j < kUnits; ++j) {
    const int64_t vi = base + j * kThreads;
    if (vi >= n_vec) return;
    const int64_t e0 = vi * 8;
    const int cnt = n - e0 >= 8 ? 8 : static_cast<int>(n - e0);
    float d[8], g[8], u[8], dg[8], du[8];
    cm::Vec8<DT, ALIGNED, true>::load(dy + e0, d, cnt);
    cm::Vec8<GT, ALIGNED, true>::load(gate + e0, g, cnt);
    if (want_dgate) cm::Vec8<UT, ALIGNED, true>::load(up + e0, u, cnt);
    silu_mul_grad8<GT>(d, g, u, dg, du, want_dgate, round_silu);
    // Both gradients are computed before either store (in-place safe).
    if (want_dgate) cm::Vec8<GT, ALIGNED>::store(dgate + e0, dg, cnt);
    if (want_dup) cm::Vec8<UT, ALIGNED>::store(dup + e0, du, cnt);
  }
}

// Row-strided forms for gate and up read from one [rows, ld_gu] buffer (the two halves of a
// merged gate/up product): row r of gate at gate + r * ld_gu, of up at up + r * ld_gu, of out
// (or dy) at + r * ld_out. cols is a multiple of 8 and every row starts 16-byte aligned, so a
// lane's 8-element vector never straddles rows: vector v is row v / vpr, columns
// 8 (v % vpr) .. +7, vpr = cols / 8 vectors per row.
template <typename GT, typename UT, typename OT>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_rows_kernel(
    const GT* __restrict__ gate, const UT* __restrict__ up, int64_t ld_gu, OT* __restrict__ out,
    int64_t ld_out, uint32_t vpr, uint32_t n_vec, int round_silu) {
  const uint32_t v = blockIdx.x * kThreads + threadIdx.x;
  if (v >= n_vec) return;
  const uint32_t r = v / vpr, c = (v - r * vpr) * 8;
  const int64_t in = static_cast<int64_t>(r) * ld_gu + c;
  float g[8], u[8], o[8];
  cm::Vec8<GT, true, true>::load(gate + in, g, 8);
  cm::Vec8<UT, true, true>::load(up + in, u, 8);
  silu_mul8<GT>(g, u, o, round_silu);
  cm::Vec8<OT, true>::store(out + static_cast<int64_t>(r) * ld_out + c, o, 8);
}

// dgate may alias gate and dup may alias up (same row stride ld_gu): no __restrict__ on those.
template <typename DT, typename GT, typename UT>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_rows_kernel(
    const DT* __restrict__ dy, int64_t ld_dy, const GT* gate, const UT* up, int64_t ld_gu,
    GT* dgate, UT* dup, uint32_t vpr, uint32_t n_vec, int want_dgate, int want_dup,
    int round_silu) {
  const uint32_t v = blockIdx.x * kThreads + threadIdx.x;
  if (v >= n_vec) return;
  const uint32_t r = v / vpr, c = (v - r * vpr) * 8;
  const int64_t in = static_cast<int64_t>(r) * ld_gu + c;
  float d[8], g[8], u[8], dg[8], du[8];
  cm::Vec8<DT, true, true>::load(dy + static_cast<int64_t>(r) * ld_dy + c, d, 8);
  cm::Vec8<GT, true, true>::load(gate + in, g, 8);
  if (want_dgate) cm::Vec8<UT, true, true>::load(up + in, u, 8);
  silu_mul_grad8<GT>(d, g, u, dg, du, want_dgate, round_silu);
  if (want_dgate) cm::Vec8<GT, true>::store(dgate + in, dg, 8);
  if (want_dup) cm::Vec8<UT, true>::store(dup + in, du, 8);
}

int64_t grid_for(int64_t n) {
  const int64_t n_vec = (n + 7) / 8;
  const int64_t per_block = int64_t{kThreads} * kUnits;
  return (n_vec + per_block - 1) / per_block;
}

bool all_aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && !cm::aligned(p, 16)) return false;
  return true;
}

}  // namespace

extern "C" int cm_swiglu_fwd(const void* gate, int g_dtype, const void* up, int u_dtype,
                             void* out, int out_dtype, int64_t n, int round_silu,
                             void* stream) {
  CM_CHECK_ARG(n >= 0);
  if (n == 0) return 0;
  CM_CHECK_ARG(gate && up && out);
  const int64_t blocks = grid_for(n);
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool al = all_aligned16({gate, up, out});
  CM_FLOAT_SWITCH(g_dtype, GT, CM_FLOAT_SWITCH(u_dtype, UT, CM_FLOAT_SWITCH(out_dtype, OT, {
    if (al)
      hipLaunchKernelGGL((swiglu_fwd_kernel<GT, UT, OT, true>), dim3(blocks), dim3(kThreads), 0,
                         s, static_cast<const GT*>(gate), static_cast<const UT*>(up),
                         static_cast<OT*>(out), n, round_silu);
    else
      hipLaunchKernelGGL((swiglu_fwd_kernel<GT, UT, OT, false>), dim3(blocks), dim3(kThreads),
                         0, s, static_cast<const GT*>(gate), static_cast<const UT*>(up),
                         static_cast<OT*>(out), n, round_silu);
  })));
  return cm::launch_status();
}

extern "C" int cm_swiglu_bwd(const void* dy, int dy_dtype, const void* gate, int g_dtype,
                             const void* up, int u_dtype, void* dgate, void* dup, int64_t n,
                             int want_dgate, int want_dup, int round_silu, void* stream) {
  CM_CHECK_ARG(n >= 0);
  if (n == 0 || !(want_dgate || want_dup)) return 0;
  CM_CHECK_ARG(dy && gate && up);
  CM_CHECK_ARG(!want_dgate || dgate);
  CM_CHECK_ARG(!want_dup || dup);
  const int64_t blocks = grid_for(n);
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool al = all_aligned16({dy, gate, up, dgate, dup});
  CM_FLOAT_SWITCH(dy_dtype, DT, CM_FLOAT_SWITCH(g_dtype, GT, CM_FLOAT_SWITCH(u_dtype, UT, {
    if (al)
      hipLaunchKernelGGL((swiglu_bwd_kernel<DT, GT, UT, true>), dim3(blocks), dim3(kThreads), 0,
                         s, static_cast<const DT*>(dy), static_cast<const GT*>(gate),
                         static_cast<const UT*>(up), static_cast<GT*>(dgate),
                         static_cast<UT*>(dup), n, want_dgate, want_dup, round_silu);
    else
      hipLaunchKernelGGL((swiglu_bwd_kernel<DT, GT, UT, false>), dim3(blocks), dim3(kThreads),
                         0, s, static_cast<const DT*>(dy), static_cast<const GT*>(gate),
                         static_cast<const UT*>(up), static_cast<GT*>(dgate),
                         static_cast<UT*>(dup), n, want_dgate, want_dup, round_silu);
  })));
  return cm::launch_status();
}

namespace {

// Shapes the row-strided kernels take: 8-element vectors that stay inside their rows, 16-byte
// aligned rows, and a vector count that fits 32 bits.
bool rows_ok(int64_t rows, int64_t cols, std::initializer_list<int64_t> lds) {
  if (rows < 0 || cols < 0 || cols % 8) return false;
  for (int64_t ld : lds)
    if (ld < cols || ld % 8) return false;
  return rows * (cols / 8) < (int64_t{1} << 32) - kThreads;
}

}  // namespace

extern "C" int cm_swiglu_fwd_rows(const void* gate, int g_dtype, const void* up, int u_dtype,
                                  int64_t ld_gu, void* out, int out_dtype, int64_t ld_out,
                                  int64_t rows, int64_t cols, int round_silu, void* stream) {
  CM_CHECK_ARG(rows_ok(rows, cols, {ld_gu, ld_out}));
  if (rows == 0 || cols == 0) return 0;
  CM_CHECK_ARG(gate && up && out && all_aligned16({gate, up, out}));
  const uint32_t vpr = static_cast<uint32_t>(cols / 8);
  const uint32_t n_vec = static_cast<uint32_t>(rows * vpr);
  const dim3 grid((n_vec + kThreads - 1) / kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  CM_FLOAT_SWITCH(g_dtype, GT, CM_FLOAT_SWITCH(u_dtype, UT, CM_FLOAT_SWITCH(out_dtype, OT, {
    hipLaunchKernelGGL((swiglu_fwd_rows_kernel<GT, UT, OT>), grid, dim3(kThreads), 0, s,
                       static_cast<const GT*>(gate), static_cast<const UT*>(up), ld_gu,
                       static_cast<OT*>(out), ld_out, vpr, n_vec, round_silu);
  })));
  return cm::launch_status();
}

extern "C" int cm_swiglu_bwd_rows(const void* dy, int dy_dtype, int64_t ld_dy, const void* gate,
                                  int g_dtype, const void* up, int u_dtype, int64_t ld_gu,
                                  void* dgate, void* dup, int64_t rows, int64_t cols,
                                  int want_dgate, int want_dup, int round_silu, void* stream) {
  CM_CHECK_ARG(rows_ok(rows, cols, {ld_dy, ld_gu}));
  if (rows == 0 || cols == 0 || !(want_dgate || want_dup)) return 0;
  CM_CHECK_ARG(dy && gate && up);
  CM_CHECK_ARG(!want_dgate || dgate);
  CM_CHECK_ARG(!want_dup || dup);
  CM_CHECK_ARG(all_aligned16({dy, gate, up, dgate, dup}));
  const uint32_t vpr = static_cast<uint32_t>(cols / 8);
  const uint32_t n_vec = static_cast<uint32_t>(rows * vpr);
  const dim3 grid((n_vec + kThreads - 1) / kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  CM_FLOAT_SWITCH(dy_dtype, DT, CM_FLOAT_SWITCH(g_dtype, GT, CM_FLOAT_SWITCH(u_dtype, UT, {
    hipLaunchKernelGGL((swiglu_bwd_rows_kernel<DT, GT, UT>), grid, dim3(kThreads), 0, s,
                       static_cast<const DT*>(dy), ld_dy, static_cast<const GT*>(gate),
                       static_cast<const UT*>(up), ld_gu, static_cast<GT*>(dgate),
                       static_cast<UT*>(dup), vpr, n_vec, want_dgate, want_dup, round_silu);
  })));
  return cm::launch_status();
}
