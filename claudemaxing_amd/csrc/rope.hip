// Rotary position embedding, forward and backward, q and k in one launch (gfx950).
//
// Reproduces solution/rope.py:17-43 (qwen_rope_kernel), which the reference launches once for
// q and once for k (rope.py:60-76). With h = D/2, x1 = x[:h], x2 = x[h:], c/s the cos/sin row
// of the token:
//   forward  o1 = x1*c1 - x2*s1,  o2 = x2*c2 + x1*s2
//   backward o1 = x1*c1 + x2*s2,  o2 = x2*c2 - x1*s1      (the transposed rotation)
// in fp32, stored in the output dtype. Inputs are strided [B, H, T, D] views (the projection
// output [B, T, H*D] transposed), outputs contiguous [B, H, T, D] or, for gradients that flow
// back into the projection, [B, T, H, D] (token-major).
//
// One workgroup handles one (batch, token): it stages that token's cos/sin rows in LDS once
// (fp32), then its lanes walk all heads of q and k (each in its own input and output dtype) in
// 4-pair groups (16-byte fp32 / 8-byte fp16
// accesses). For the Qwen2.5 layout (12 + 2 heads, D = 128) that is 14 * 16 = 224 lanes, and
// the q/k reads of a token are one contiguous span of the projection output.
#include "common.h"

namespace {

#pragma clang fp contract(off)

constexpr int kThreads = 256;
constexpr int kMaxD = 512;

template <typename T, int N>
struct VecN {
  static __device__ __forceinline__ void load(const T* p, float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = cm::to_f32(p[i]);
  }
  static __device__ __forceinline__ void store(T* p, const float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = cm::from_f32<T>(v[i]);
  }
};

template <>
struct VecN<_Float16, 4> {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ void load(const _Float16* p, float (&v)[4]) {
    const h4 h = *reinterpret_cast<const h4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = static_cast<float>(h[i]);
  }
  static __device__ __forceinline__ void store(_Float16* p, const float (&v)[4]) {
    h4 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = cm::from_f32<_Float16>(v[i]);
    *reinterpret_cast<h4*>(p) = h;
  }
};

template <>
struct VecN<float, 4> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

// One G-pair group of one head row: src / dst point at the row's first element.
template <typename XT, typename OT, int G>
__device__ __forceinline__ void rotate_group(const XT* src, OT* dst, int p0, int half,
                                             const float* s_cos, const float* s_sin,
                                             bool backward) {
  float a[G], c[G], o1[G], o2[G];
  VecN<XT, G>::load(src + p0, a);
  VecN<XT, G>::load(src + half + p0, c);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float c1 = s_cos[p0 + i], c2 = s_cos[half + p0 + i];
    const float s1 = s_sin[p0 + i], s2 = s_sin[half + p0 + i];
    if (backward) {
      o1[i] = a[i] * c1 + c[i] * s2;
      o2[i] = c[i] * c2 - a[i] * s1;
    } else {
      o1[i] = a[i] * c1 - c[i] * s1;
      o2[i] = c[i] * c2 + a[i] * s2;
    }
  }
  VecN<OT, G>::store(dst + p0, o1);
  VecN<OT, G>::store(dst + half + p0, o2);
}

// Tensor 0 is read as X0 and written as O0, tensor 1 as X1 / O1 (the training step's q and k
// differ: fp32 q and fp16 k forward, fp32 and fp16 gradients backward).
template <typename X0, typename O0, typename X1, typename O1, typename CT, int G>
__global__ __launch_bounds__(kThreads) void rope_kernel(
    const X0* __restrict__ x0, int64_t sb0, int64_t sh0, int64_t st0, int H0,
    O0* __restrict__ out0, const X1* __restrict__ x1, int64_t sb1, int64_t sh1, int64_t st1,
    int H1, O1* __restrict__ out1, const CT* __restrict__ cos, const CT* __restrict__ sin,
    int64_t cs_b, int64_t cs_t, int T, int D, int flags) {
  const bool backward = flags & 1;
  __shared__ float s_cos[kMaxD];
  __shared__ float s_sin[kMaxD];
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const int64_t crow = static_cast<int64_t>(b) * cs_b + static_cast<int64_t>(t) * cs_t;
  for (int d = threadIdx.x; d < D; d += kThreads) {
    s_cos[d] = cm::to_f32(cos[crow + d]);
    s_sin[d] = cm::to_f32(sin[crow + d]);
  }
  __syncthreads();
  const int half = D / 2;
  const int groups = half / G;  // G-pair groups per head
  const int total = (H0 + H1) * groups;
  // output row of head h of H: [B][H][T][D], or [B][T][H][D] with bit 1 of flags
  auto out_row = [&](int h, int H) {
    return ((flags & 2) ? (static_cast<int64_t>(b) * T + t) * H + h
                        : (static_cast<int64_t>(b) * H + h) * T + t) *
           static_cast<int64_t>(D);
  };
  for (int w = threadIdx.x; w < total; w += kThreads) {
    int h = w / groups;
    const int p0 = (w - h * groups) * G;
    if (h < H0) {
      rotate_group<X0, O0, G>(x0 + static_cast<int64_t>(b) * sb0 + static_cast<int64_t>(h) * sh0 +
                                  static_cast<int64_t>(t) * st0,
                              out0 + out_row(h, H0), p0, half, s_cos, s_sin, backward);
    } else {
      h -= H0;
      rotate_group<X1, O1, G>(x1 + static_cast<int64_t>(b) * sb1 + static_cast<int64_t>(h) * sh1 +
                                  static_cast<int64_t>(t) * st1,
                              out1 + out_row(h, H1), p0, half, s_cos, s_sin, backward);
    }
  }
}

template <typename X0, typename O0, typename X1, typename O1, typename CT>
int launch_typed(const void* x0, int64_t sb0, int64_t sh0, int64_t st0, int H0, void* out0,
                 const void* x1, int64_t sb1, int64_t sh1, int64_t st1, int H1, void* out1,
                 const void* cos, const void* sin, int64_t cs_b, int64_t cs_t, int B, int T,
                 int D, int flags, hipStream_t s) {
  dim3 grid(T, B);
  const int half = D / 2;
  // 4-pair groups when each group start is a multiple of 4 elements (strides and D allow it).
  // Base pointers must then be aligned to 4 elements for the vector accesses.
  const bool g4 = half % 4 == 0 && sh0 % 4 == 0 && st0 % 4 == 0 && sb0 % 4 == 0 &&
                  cm::aligned(x0, 4 * sizeof(X0)) && cm::aligned(out0, 4 * sizeof(O0)) &&
                  (H1 == 0 || (sh1 % 4 == 0 && st1 % 4 == 0 && sb1 % 4 == 0 &&
                               cm::aligned(x1, 4 * sizeof(X1)) &&
                               cm::aligned(out1, 4 * sizeof(O1))));
#define CM_ROPE_LAUNCH(G)                                                                      \
  hipLaunchKernelGGL((rope_kernel<X0, O0, X1, O1, CT, G>), grid, dim3(kThreads), 0, s,         \
                     static_cast<const X0*>(x0), sb0, sh0, st0, H0, static_cast<O0*>(out0),    \
                     static_cast<const X1*>(x1), sb1, sh1, st1, H1, static_cast<O1*>(out1),    \
                     static_cast<const CT*>(cos), static_cast<const CT*>(sin), cs_b, cs_t, T, D, \
                     flags)
  if (g4)
    CM_ROPE_LAUNCH(4);
  else
    CM_ROPE_LAUNCH(1);
#undef CM_ROPE_LAUNCH
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_rope(const void* x0, int x0_dtype, int64_t sb0, int64_t sh0, int64_t st0,
                       int H0, void* out0, int out0_dtype, const void* x1, int x1_dtype,
                       int64_t sb1, int64_t sh1, int64_t st1, int H1, void* out1,
                       int out1_dtype, const void* cos, const void* sin, int cs_dtype,
                       int64_t cs_b, int64_t cs_t, int B, int T, int D, int flags,
                       void* stream) {
  CM_CHECK_ARG(B >= 0 && T >= 0 && H0 >= 0 && H1 >= 0);
  CM_CHECK_ARG(D > 0 && D % 2 == 0 && D <= kMaxD);
  CM_CHECK_ARG(flags >= 0 && flags <= 3);
  if (B == 0 || T == 0 || H0 + H1 == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff && B <= 65535);
  CM_CHECK_ARG(cos && sin);
  CM_CHECK_ARG(H0 == 0 || (x0 && out0));
  CM_CHECK_ARG(H1 == 0 || (x1 && out1));
  hipStream_t s = static_cast<hipStream_t>(stream);
  // One launch covers both tensors when their dtypes agree, and for the training step's mixed
  // pairs with fp32 cos/sin (fp32 q with fp16 k forward: both written fp32; fp32 q and k
  // gradients written fp32 and fp16 backward); otherwise one launch each.
  if (H0 > 0 && H1 > 0 && cs_dtype == CM_F32 && x0_dtype == CM_F32 && out0_dtype == CM_F32) {
    if (x1_dtype == CM_F16 && out1_dtype == CM_F32) {
      return launch_typed<float, float, _Float16, float, float>(
          x0, sb0, sh0, st0, H0, out0, x1, sb1, sh1, st1, H1, out1, cos, sin, cs_b, cs_t, B, T,
          D, flags, s);
    }
    if (x1_dtype == CM_F32 && out1_dtype == CM_F16) {
      return launch_typed<float, float, float, _Float16, float>(
          x0, sb0, sh0, st0, H0, out0, x1, sb1, sh1, st1, H1, out1, cos, sin, cs_b, cs_t, B, T,
          D, flags, s);
    }
  }
  if (H0 > 0 && H1 > 0 && (x0_dtype != x1_dtype || out0_dtype != out1_dtype)) {
    int st = cm_rope(x0, x0_dtype, sb0, sh0, st0, H0, out0, out0_dtype, nullptr, x0_dtype, 0, 0,
                     0, 0, nullptr, out0_dtype, cos, sin, cs_dtype, cs_b, cs_t, B, T, D,
                     flags, stream);
    if (st) return st;
    return cm_rope(x1, x1_dtype, sb1, sh1, st1, H1, out1, out1_dtype, nullptr, x1_dtype, 0, 0, 0,
                   0, nullptr, out1_dtype, cos, sin, cs_dtype, cs_b, cs_t, B, T, D, flags,
                   stream);
  }
  if (H0 == 0) {  // single tensor passed in the second slot: move it to the first
    return cm_rope(x1, x1_dtype, sb1, sh1, st1, H1, out1, out1_dtype, nullptr, x1_dtype, 0, 0, 0,
                   0, nullptr, out1_dtype, cos, sin, cs_dtype, cs_b, cs_t, B, T, D, flags,
                   stream);
  }
  CM_FLOAT_SWITCH(x0_dtype, XT, CM_FLOAT_SWITCH(out0_dtype, OT, CM_FLOAT_SWITCH(cs_dtype, CT, {
    return launch_typed<XT, OT, XT, OT, CT>(x0, sb0, sh0, st0, H0, out0, x1, sb1, sh1, st1, H1,
                                            out1, cos, sin, cs_b, cs_t, B, T, D, flags, s);
  })));
  return 0;
}
