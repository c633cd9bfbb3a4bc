// A LoRA adapter of rank 16 on a frozen base projection, fused per token row (gfx950).
//
// The reference computes the adapter with torch around its two mask kernels (solution/lora.py:
// LoRABranch 78-107, the pack/unpack kernels 30-57): per call the two fp32 adapter weights are
// cast to fp16, lora_B(lora_A(xd)) runs as two rank-16 GEMMs, the result is scaled, widened and
// added to the base output, and the backward runs four more GEMMs, casts and the unpack. At the
// QLoRA step's sizes (1276 tokens, width 1536) each of those is a few-microsecond launch. Here
// one kernel per direction handles everything that is local to a token row; only the two
// weight-gradient products, which sum over the tokens, stay GEMMs.
//
// Forward, row t (K inputs, N outputs, R = 16):
//   xd   = fp16(keep ? x * scale_p : 0)                     (the pack kernel, bit for bit)
//   a    = fp16(sum_k xd[k] * fp16(A)[r][k])                 (lora_A, fp32 accumulation)
//   lora = fp16(fp16(sum_r a[r] * fp16(B)[n][r]) * scaling)   (lora_B, then the scaling)
//   out  = fp32(base16[n]) + fp32(lora)                       (widen, add to the base output)
// writing out, the mask bits and a (saved for the backward).
// Backward-1, row t: gbase = fp16(grad) (the base output's widening, backwards);
//   g = fp16(gbase * scaling); ga = fp16(sum_n g[n] * fp16(B)[n][r]).
// Backward-2, row t, after the caller's base input gradient dxb = gbase @ W (fp16):
//   gxd = fp16(sum_r ga[r] * fp16(A)[r][k]);
//   dx  = fp32(dxb[k]) + (keep ? gxd * scale_p : 0)           (the unpack kernel's gradient)
//   or, without dxb, dx += (keep ? gxd * scale_p : 0)         (a second adapter on the same input)
//   xd' = fp16(keep ? x16 * scale_p : 0)                       (lora_A's input, rebuilt)
// The products of two fp16 values are exact in fp32, so the sums differ from a GEMM's only in
// their order.
//
// Work split: a workgroup of 256 lanes handles kRows rows; lane c owns the 8 inputs 8c..8c+7
// (the fp16 adapter weights of its columns stay in registers for all rows) and the outputs
// c + 256 j. A row's inputs are loaded while the previous row is computed (the rows of a
// workgroup would otherwise each wait out a full memory latency). The rank-16 reductions over
// K (or N) are a halving shuffle butterfly per wavefront and a 4-way LDS sum.
#include "common.h"

namespace {

#pragma clang fp contract(off)

constexpr int kThreads = 256;
constexpr int kR = 16;       // LoRA rank
constexpr int kMaxNJ = 8;    // outputs per lane: N <= 2048
#ifndef CM_LORA_ROWS
#define CM_LORA_ROWS 4
#endif
constexpr int kRows = CM_LORA_ROWS;  // token rows per workgroup (4: 31.0 ms graphed step; 2: 31.5, 8: 31.8, 16: 33.5)
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ _Float16 h16(float v) { return cm::from_f32<_Float16>(v); }

// 16 per-lane partial sums reduced over the workgroup; thread r < 16 returns sum r. Within a
// wavefront the reduction halves the values it exchanges at each step (lanes l and l ^ 32 swap
// the halves they do not keep, then l ^ 16, l ^ 8, l ^ 4): 8 + 4 + 2 + 1 shuffles, after which
// lane l holds rank ((l >> 5) & 1) * 8 + ((l >> 4) & 1) * 4 + ((l >> 3) & 1) * 2 + ((l >> 2) & 1)
// summed over 16 lanes; two more shuffles finish the quad. The 4 wavefronts meet in LDS.
__device__ __forceinline__ float block_sum16(float (&p)[kR], float (*red)[kR], int lane,
                                             int wave) {
  float q8[8], q4[4], q2[2];
  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8, b2 = lane & 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float mine = b5 ? p[8 + i] : p[i], other = b5 ? p[i] : p[8 + i];
    q8[i] = mine + __shfl_xor(other, 32, cm::kWave);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float mine = b4 ? q8[4 + i] : q8[i], other = b4 ? q8[i] : q8[4 + i];
    q4[i] = mine + __shfl_xor(other, 16, cm::kWave);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float mine = b3 ? q4[2 + i] : q4[i], other = b3 ? q4[i] : q4[2 + i];
    q2[i] = mine + __shfl_xor(other, 8, cm::kWave);
  }
  float v;
  {
    const float mine = b2 ? q2[1] : q2[0], other = b2 ? q2[0] : q2[1];
    v = mine + __shfl_xor(other, 4, cm::kWave);
  }
  v += __shfl_xor(v, 2, cm::kWave);
  v += __shfl_xor(v, 1, cm::kWave);
  if ((lane & 3) == 0) red[wave][(b5 ? 8 : 0) + (b4 ? 4 : 0) + (b3 ? 2 : 0) + (b2 ? 1 : 0)] = v;
  __syncthreads();
  float s = 0.0f;
  if (threadIdx.x < kR) s = (red[0][threadIdx.x] + red[1][threadIdx.x]) +
                            (red[2][threadIdx.x] + red[3][threadIdx.x]);
  return s;
}

// fp16(A)[r][8c .. 8c+7] for r < 16 (zero past K).
__device__ __forceinline__ void load_a16(const float* A, int K, int c, half8 (&a)[kR]) {
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    if (8 * c < K) {
      const float4* p = reinterpret_cast<const float4*>(A + static_cast<int64_t>(r) * K + 8 * c);
      const float4 u = p[0], v = p[1];
      a[r][0] = h16(u.x); a[r][1] = h16(u.y); a[r][2] = h16(u.z); a[r][3] = h16(u.w);
      a[r][4] = h16(v.x); a[r][5] = h16(v.y); a[r][6] = h16(v.z); a[r][7] = h16(v.w);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[r][i] = static_cast<_Float16>(0.0f);
    }
  }
}

// fp16(B)[n][0 .. 15] for the lane's outputs n = c + 256 j (zero past N).
template <int NJ>
__device__ __forceinline__ void load_b16(const float* B, int N, int c, _Float16 (&b)[NJ][kR]) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = c + kThreads * j;
#pragma unroll
    for (int q = 0; q < kR / 4; ++q) {
      const float4 v = n < N ? reinterpret_cast<const float4*>(B + static_cast<int64_t>(n) * kR)[q]
                             : make_float4(0.f, 0.f, 0.f, 0.f);
      b[j][4 * q] = h16(v.x); b[j][4 * q + 1] = h16(v.y);
      b[j][4 * q + 2] = h16(v.z); b[j][4 * q + 3] = h16(v.w);
    }
  }
}

template <int NJ>
__global__ __launch_bounds__(kThreads) void lora_fused_fwd_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ keep, const float* __restrict__ A,
    const float* __restrict__ B, const _Float16* __restrict__ base, float* __restrict__ out,
    uint8_t* __restrict__ bits, _Float16* __restrict__ a16, int T, int K, int N,
    float scale_p, float scaling) {
  __shared__ float red[kThreads / cm::kWave][kR];
  __shared__ float arow[kR];
  const int c = threadIdx.x, lane = c % cm::kWave, wave = c / cm::kWave;
  const bool kok = 8 * c < K;
  const int t0 = blockIdx.x * kRows, t_end = min(T, t0 + kRows);
  // the row's inputs, loaded one row ahead of their use
  struct In {
    float4 u, v;
    uint2 kk;
    _Float16 b[NJ];
  };
  auto load = [&](int t, In& in) {
    if (kok) {
      const int64_t at = static_cast<int64_t>(t) * K + 8 * c;
      in.u = reinterpret_cast<const float4*>(x + at)[0];
      in.v = reinterpret_cast<const float4*>(x + at)[1];
      in.kk = *reinterpret_cast<const uint2*>(keep + at);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = c + kThreads * j;
      in.b[j] = n < N ? base[static_cast<int64_t>(t) * N + n] : static_cast<_Float16>(0.0f);
    }
  };
  In cur, nxt;
  load(t0, cur);
  half8 ar[kR];
  load_a16(A, K, c, ar);
  _Float16 br[NJ][kR];
  load_b16<NJ>(B, N, c, br);
  for (int t = t0; t < t_end; ++t) {
    if (t + 1 < t_end) load(t + 1, nxt);
    float p[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) p[r] = 0.0f;
    if (kok) {
      const float xv[8] = {cur.u.x, cur.u.y, cur.u.z, cur.u.w, cur.v.x, cur.v.y, cur.v.z, cur.v.w};
      float xd[8];
      uint32_t byte = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool kept = (((i < 4 ? cur.kk.x : cur.kk.y) >> (8 * (i & 3))) & 0xffu) != 0;
        byte |= static_cast<uint32_t>(kept) << i;
        xd[i] = static_cast<float>(h16(kept ? xv[i] * scale_p : 0.0f));
      }
      bits[static_cast<int64_t>(t) * (K / 8) + c] = static_cast<uint8_t>(byte);
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += xd[i] * static_cast<float>(ar[r][i]);
        p[r] = s;
      }
    }
    const float s = block_sum16(p, red, lane, wave);
    if (c < kR) {
      const _Float16 h = h16(s);
      a16[static_cast<int64_t>(t) * kR + c] = h;
      arow[c] = static_cast<float>(h);
    }
    __syncthreads();
    float av[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) av[r] = arow[r];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = c + kThreads * j;
      if (n >= N) break;
      float o = 0.0f;
#pragma unroll
      for (int r = 0; r < kR; ++r) o += av[r] * static_cast<float>(br[j][r]);
      const float lora = static_cast<float>(h16(static_cast<float>(h16(o)) * scaling));
      out[static_cast<int64_t>(t) * N + n] = static_cast<float>(cur.b[j]) + lora;
    }
    __syncthreads();  // red / arow are rewritten by the next row
    cur = nxt;
  }
}

template <int NJ>
__global__ __launch_bounds__(kThreads) void lora_fused_bwd1_kernel(
    const float* __restrict__ grad, const float* __restrict__ B, _Float16* __restrict__ gbase,
    _Float16* __restrict__ g16, _Float16* __restrict__ ga16, int T, int N, float scaling) {
  __shared__ float red[kThreads / cm::kWave][kR];
  const int c = threadIdx.x, lane = c % cm::kWave, wave = c / cm::kWave;
  const int t0 = blockIdx.x * kRows, t_end = min(T, t0 + kRows);
  float cur[NJ], nxt[NJ];
  auto load = [&](int t, float (&g)[NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = c + kThreads * j;
      g[j] = n < N ? grad[static_cast<int64_t>(t) * N + n] : 0.0f;
    }
  };
  load(t0, cur);
  _Float16 br[NJ][kR];
  load_b16<NJ>(B, N, c, br);
  for (int t = t0; t < t_end; ++t) {
    if (t + 1 < t_end) load(t + 1, nxt);
    float p[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) p[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = c + kThreads * j;
      if (n >= N) break;
      const int64_t at = static_cast<int64_t>(t) * N + n;
      const _Float16 gb = h16(cur[j]);
      const _Float16 g = h16(static_cast<float>(gb) * scaling);
      gbase[at] = gb;
      g16[at] = g;
      const float gf = static_cast<float>(g);
#pragma unroll
      for (int r = 0; r < kR; ++r) p[r] += gf * static_cast<float>(br[j][r]);
    }
    const float s = block_sum16(p, red, lane, wave);
    if (c < kR) ga16[static_cast<int64_t>(t) * kR + c] = h16(s);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) cur[j] = nxt[j];
  }
}

__global__ __launch_bounds__(kThreads) void lora_fused_bwd2_kernel(
    const _Float16* __restrict__ dxb, const _Float16* __restrict__ ga16,
    const float* __restrict__ A, const _Float16* __restrict__ x16,
    const uint8_t* __restrict__ bits, float* __restrict__ dx, _Float16* __restrict__ xd16,
    int T, int K, float scale_p) {
  const int c = threadIdx.x;
  if (8 * c >= K) return;  // no barrier below
  const int t0 = blockIdx.x * kRows, t_end = min(T, t0 + kRows);
  struct In {
    half8 ga0, ga1, db, xv;
    float4 d0, d1;  // dx as it is (accumulating)
    uint32_t m;
  };
  auto load = [&](int t, In& in) {
    const int64_t at = static_cast<int64_t>(t) * K + 8 * c;
    in.ga0 = *reinterpret_cast<const half8*>(ga16 + static_cast<int64_t>(t) * kR);
    in.ga1 = *reinterpret_cast<const half8*>(ga16 + static_cast<int64_t>(t) * kR + 8);
    if (dx && dxb) {
      in.db = *reinterpret_cast<const half8*>(dxb + at);
    } else if (dx) {
      in.d0 = reinterpret_cast<const float4*>(dx + at)[0];
      in.d1 = reinterpret_cast<const float4*>(dx + at)[1];
    }
    in.xv = *reinterpret_cast<const half8*>(x16 + at);
    in.m = bits[static_cast<int64_t>(t) * (K / 8) + c];
  };
  In cur, nxt;
  load(t0, cur);
  half8 ar[kR];
  load_a16(A, K, c, ar);
  for (int t = t0; t < t_end; ++t) {
    if (t + 1 < t_end) load(t + 1, nxt);
    const int64_t at = static_cast<int64_t>(t) * K + 8 * c;
    float gxd[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) gxd[i] = 0.0f;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const float g = static_cast<float>(r < 8 ? cur.ga0[r] : cur.ga1[r - 8]);
#pragma unroll
      for (int i = 0; i < 8; ++i) gxd[i] += g * static_cast<float>(ar[r][i]);
    }
    float o[8];
    half8 xo;
    const float dold[8] = {cur.d0.x, cur.d0.y, cur.d0.z, cur.d0.w,
                           cur.d1.x, cur.d1.y, cur.d1.z, cur.d1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool kept = (cur.m >> i) & 1u;
      const float gl = kept ? static_cast<float>(h16(gxd[i])) * scale_p : 0.0f;
      o[i] = dx ? (dxb ? static_cast<float>(cur.db[i]) : dold[i]) + gl : 0.0f;
      xo[i] = h16(kept ? static_cast<float>(cur.xv[i]) * scale_p : 0.0f);
    }
    if (dx) {
      float4* d = reinterpret_cast<float4*>(dx + at);
      d[0] = make_float4(o[0], o[1], o[2], o[3]);
      d[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
    *reinterpret_cast<half8*>(xd16 + at) = xo;
    cur = nxt;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

#define CM_LORA_NJ_SWITCH(nj, NJ, ...)           \
  switch (nj) {                                  \
    case 1: { constexpr int NJ = 1; __VA_ARGS__; break; } \
    case 2: { constexpr int NJ = 2; __VA_ARGS__; break; } \
    case 4: { constexpr int NJ = 4; __VA_ARGS__; break; } \
    case 6: { constexpr int NJ = 6; __VA_ARGS__; break; } \
    default: { constexpr int NJ = 8; __VA_ARGS__; break; } \
  }

namespace {
int nj_for(int n) {
  const int nj = (n + kThreads - 1) / kThreads;
  return nj <= 1 ? 1 : nj <= 2 ? 2 : nj <= 4 ? 4 : nj <= 6 ? 6 : 8;
}
}  // namespace

extern "C" int cm_lora_fused_fwd(const float* x, const uint8_t* keep, const float* weight_a,
                                 const float* weight_b, const void* base16, float* out,
                                 uint8_t* bits, void* a16, int64_t T, int K, int N, int rank,
                                 float scale_p, float scaling, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && K > 0 && N > 0);
  CM_CHECK_ARG(K % 8 == 0 && K <= 8 * kThreads && N <= kMaxNJ * kThreads);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  CM_CHECK_ARG(x && keep && weight_a && weight_b && base16 && out && bits && a16);
  CM_CHECK_ARG(aligned16(x) && (reinterpret_cast<uintptr_t>(keep) & 7) == 0 &&
               aligned16(weight_a) && aligned16(weight_b));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((T + kRows - 1) / kRows));
  CM_LORA_NJ_SWITCH(nj_for(N), NJ, {
    hipLaunchKernelGGL(lora_fused_fwd_kernel<NJ>, grid, dim3(kThreads), 0, s, x, keep, weight_a,
                       weight_b, static_cast<const _Float16*>(base16), out, bits,
                       static_cast<_Float16*>(a16), static_cast<int>(T), K, N, scale_p, scaling);
  });
  return cm::launch_status();
}

extern "C" int cm_lora_fused_bwd1(const float* grad, const float* weight_b, void* gbase16,
                                  void* g16, void* ga16, int64_t T, int N, int rank,
                                  float scaling, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && N > 0 && N <= kMaxNJ * kThreads);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  CM_CHECK_ARG(grad && weight_b && gbase16 && g16 && ga16 && aligned16(weight_b));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((T + kRows - 1) / kRows));
  CM_LORA_NJ_SWITCH(nj_for(N), NJ, {
    hipLaunchKernelGGL(lora_fused_bwd1_kernel<NJ>, grid, dim3(kThreads), 0, s, grad, weight_b,
                       static_cast<_Float16*>(gbase16), static_cast<_Float16*>(g16),
                       static_cast<_Float16*>(ga16), static_cast<int>(T), N, scaling);
  });
  return cm::launch_status();
}

extern "C" int cm_lora_fused_bwd2(const void* dxb16, const void* ga16, const float* weight_a,
                                  const void* x16, const uint8_t* bits, float* dx, void* xd16,
                                  int64_t T, int K, int rank, float scale_p, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && K > 0 && K % 8 == 0 && K <= 8 * kThreads);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  CM_CHECK_ARG(ga16 && weight_a && x16 && bits && xd16);
  CM_CHECK_ARG((!dx || ((!dxb16 || aligned16(dxb16)) && aligned16(dx))) && aligned16(ga16) &&
               aligned16(weight_a) && aligned16(x16) && aligned16(xd16));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((T + kRows - 1) / kRows));
  hipLaunchKernelGGL(lora_fused_bwd2_kernel, grid, dim3(kThreads), 0, s,
                     static_cast<const _Float16*>(dxb16), static_cast<const _Float16*>(ga16),
                     weight_a, static_cast<const _Float16*>(x16), bits, dx,
                     static_cast<_Float16*>(xd16), static_cast<int>(T), K, scale_p);
  return cm::launch_status();
}
