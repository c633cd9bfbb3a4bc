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
// Work split: a workgroup of 8 wavefronts takes a tile of up to 16 token rows (the host picks
// fewer rows per tile when that spreads a small batch over more CUs). The rank-16 products run
// on the matrix cores with fp16 operands and fp32 accumulation, like the GEMMs they replace:
// the sums over K (or N) as v_mfma_f32_16x16x32_f16 steps of 32, split over the wavefronts and
// added in a fixed order through the LDS; the expansions back to N (or K) outputs as one
// v_mfma_f32_16x16x16_f16 per 16 outputs, split over the wavefronts. Operands are assigned to
// lanes so that each lane's memory accesses are 8 to 32 contiguous bytes, and a wavefront issues
// all its loads before its first product: a launch costs about one memory round trip plus its
// stores, the arithmetic being a few dozen matrix instructions per wavefront.
//
// 16x16 MFMA tiles: lane l supplies row l % 16 of the left operand and column l % 16 of the right
// one, both over the k values of lane group g = l / 16 (8 of 32 for 16x16x32, 4 of 16 for
// 16x16x16), and receives rows 4 g .. 4 g + 3 of column l % 16 of the result. Which 8 of a step's
// 32 k values a lane group supplies is free as long as both operands agree: here k = 4 g .. 4 g + 3
// and 16 + 4 g .. 16 + 4 g + 3, so that the 4 lane groups of a row read 64 contiguous bytes per
// 16-byte access (a wavefront's access then covers 16 runs of 64 bytes; lanes 32 bytes apart
// would cost the address units a request per lane).
//
// Loads are unconditional, from addresses clamped into the arrays: rows past T (or past the
// tile, which repeat its last row) and lanes past K or N read real, finite data whose results
// are never stored, and inputs
// past K (or N) inside a sum are zeroed by a select after the loads. A load under a branch with a
// zero default would make the compiler merge the two values at the join, waiting there for the
// load, which turns one memory round trip into several.
#include "common.h"

namespace {

#pragma clang fp contract(off)

constexpr int kR = 16;         // LoRA rank
constexpr int kWaves = 8;      // wavefronts per workgroup
constexpr int kThreads = kWaves * cm::kWave;
constexpr int kTileRows = 16;  // token rows per tile at most (the MFMA tile height)
constexpr int kMaxK = 2048, kMaxN = 2048;
constexpr int kCUs = 256;      // MI355X compute units
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float acc4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ _Float16 h16(float v) { return cm::from_f32<_Float16>(v); }

__device__ __forceinline__ half8 to_half8(float4 u, float4 v) {
  half8 h;
  h[0] = h16(u.x); h[1] = h16(u.y); h[2] = h16(u.z); h[3] = h16(u.w);
  h[4] = h16(v.x); h[5] = h16(v.y); h[6] = h16(v.z); h[7] = h16(v.w);
  return h;
}

__device__ __forceinline__ acc4 mfma_k32(half8 a, half8 b, acc4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ acc4 mfma_k16(half4 a, half4 b, acc4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Value i of lane l of the 16x16 tile, summed over the 8 wavefronts' partial tiles in a fixed
// order.
__device__ __forceinline__ float sum_waves(const acc4 (*red)[cm::kWave], int l, int i) {
  float v[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) v[w] = red[w][l][i];
  return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

__device__ __forceinline__ int wave_index() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / cm::kWave);
}

// Forward. lora_A: a[rows x 16] = xd . fp16(A)^T, step s (inputs 32 s .. 32 s + 31) on wavefront
// s % 8; lane l brings row l % 16's xd at inputs 32 s + 4 g .. +3 and 32 s + 16 + 4 g .. +3 and
// fp16(A)[rank l % 16] at the same inputs; the row's 4 lane groups then assemble its 4 mask bytes
// for lane group 0 to write. lora_B: out^T[16-output tile j x rows] =
// fp16(B)[tile] . a^T, tile j on wavefront j % 8; lane l gets row l % 16 and the 4 consecutive
// outputs 16 j + 4 (l / 16) .. +3 (base read 8 bytes, out written 16 bytes at a time).
// SK and SN bound the steps and tiles per wavefront.
// One adapter's operands; a launch takes up to kMaxJobs adapters on the same input x (the q and v
// adapters of an attention block), adapter blockIdx.y, so that their independent row tiles run
// side by side instead of one launch after the other.
constexpr int kMaxJobs = 4;
struct FwdJob {
  const uint8_t* keep;
  const float* A;
  const float* B;
  const _Float16* base;
  float* out;
  uint8_t* bits;
  _Float16* a16;
  int N;
};
struct FwdJobs {
  FwdJob j[kMaxJobs];
};

template <int SK, int SN>
__global__ __launch_bounds__(kThreads) void lora_fused_fwd_kernel(
    const float* __restrict__ x, FwdJobs jobs, int T, int K, int rows, float scale_p,
    float scaling) {
  const FwdJob jb = jobs.j[blockIdx.y];
  const uint8_t* __restrict__ keep = jb.keep;
  const float* __restrict__ A = jb.A;
  const float* __restrict__ B = jb.B;
  const _Float16* __restrict__ base = jb.base;
  float* __restrict__ out = jb.out;
  uint8_t* __restrict__ bits = jb.bits;
  _Float16* __restrict__ a16 = jb.a16;
  const int N = jb.N;
  __shared__ acc4 red[kWaves][cm::kWave];
  const int lane = threadIdx.x % cm::kWave, wave = wave_index();
  const int r16 = lane % 16, grp = lane / 16;
  const int t = blockIdx.x * rows + r16;
  const bool live = r16 < rows && t < T;
  const int K8 = K / 8, steps = (K + 31) / 32, tiles = (N + 15) / 16;
  const bool words = K8 % 4 == 0 && (reinterpret_cast<uintptr_t>(bits) & 3) == 0;
  // lanes past the tile repeat its last row (the same cache lines, no extra traffic)
  const int64_t tc = min(blockIdx.x * rows + min(r16, rows - 1), T - 1);
  float4 xv[SK][2], av[SK][2];
  uint32_t kk[SK][2];
#pragma unroll
  for (int i = 0; i < SK; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = min(32 * (wave + kWaves * i) + 16 * h + 4 * grp, K - 4);
      xv[i][h] = *reinterpret_cast<const float4*>(x + tc * K + k);
      kk[i][h] = *reinterpret_cast<const uint32_t*>(keep + tc * K + k);
      av[i][h] = *reinterpret_cast<const float4*>(A + static_cast<int64_t>(r16) * K + k);
    }
  }
  uint2 bb[SN];  // fp16 base values of this lane's 4 outputs per tile
#pragma unroll
  for (int i = 0; i < SN; ++i) {
    const int n = min(16 * (wave + kWaves * i) + 4 * grp, N - 4);
    bb[i] = *reinterpret_cast<const uint2*>(base + tc * N + n);
  }
  acc4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < SK; ++i) {
    const int s = wave + kWaves * i;
    if (s >= steps) break;
    const float xs[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                         xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
    const bool in0 = 32 * s + 4 * grp < K, in1 = 32 * s + 16 + 4 * grp < K;
    half8 xd, ad;
    uint32_t nib = 0;  // bits 0-3: inputs 32 s + 4 g .., bits 4-7: 32 s + 16 + 4 g ..
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = e < 4 ? in0 : in1;
      const bool kept = in && ((kk[i][e / 4] >> (8 * (e & 3))) & 0xffu) != 0;
      nib |= static_cast<uint32_t>(kept) << e;
      xd[e] = h16(kept ? xs[e] * scale_p : 0.0f);
      const float4 a4 = av[i][e / 4];
      const float ae = (e & 3) == 0 ? a4.x : (e & 3) == 1 ? a4.y : (e & 3) == 2 ? a4.z : a4.w;
      ad[e] = h16(in ? ae : 0.0f);
    }
    // mask bytes 4 s .. 4 s + 3 of the row: byte 4 s + b holds lane groups 2 (b % 2) and
    // 2 (b % 2) + 1 of half b / 2
    const uint32_t n1 = __shfl_xor(nib, 16, cm::kWave), n2 = __shfl_xor(nib, 32, cm::kWave),
                   n3 = __shfl_xor(nib, 48, cm::kWave);
    if (grp == 0 && live) {
      const uint32_t word = (nib & 0xfu) | (n1 & 0xfu) << 4 | (n2 & 0xfu) << 8 |
                            (n3 & 0xfu) << 12 | (nib >> 4) << 16 | (n1 >> 4) << 20 |
                            (n2 >> 4) << 24 | (n3 >> 4) << 28;
      uint8_t* dst = bits + static_cast<int64_t>(t) * K8 + 4 * s;
      if (words) {
        *reinterpret_cast<uint32_t*>(dst) = word;
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (4 * s + b < K8) dst[b] = static_cast<uint8_t>(word >> (8 * b));
      }
    }
    acc = mfma_k32(xd, ad, acc);
  }
  red[wave][lane] = acc;
  float4 bq[SN];  // fp32 B[16 j + l % 16][4 (l / 16) .. +3]
#pragma unroll
  for (int i = 0; i < SN; ++i) {
    // rows past N only feed outputs past N, which are not stored
    const int n = min(16 * (wave + kWaves * i) + r16, N - 1);
    bq[i] = *reinterpret_cast<const float4*>(B + static_cast<int64_t>(n) * kR + 4 * grp);
  }
  __syncthreads();
  // a[row l % 16][ranks 4 (l / 16) .. +3]: a[m][r] is value m % 4 of lane r + 16 (m / 4)
  half4 ah;
#pragma unroll
  for (int e = 0; e < 4; ++e) ah[e] = h16(sum_waves(red, 4 * grp + e + 16 * (r16 / 4), r16 % 4));
  if (wave == 0 && live)
    *reinterpret_cast<half4*>(a16 + static_cast<int64_t>(t) * kR + 4 * grp) = ah;
#pragma unroll
  for (int i = 0; i < SN; ++i) {
    const int j = wave + kWaves * i;
    if (j >= tiles) break;
    half4 bh;
    bh[0] = h16(bq[i].x); bh[1] = h16(bq[i].y); bh[2] = h16(bq[i].z); bh[3] = h16(bq[i].w);
    const acc4 o = mfma_k16(bh, ah, acc4{0.f, 0.f, 0.f, 0.f});
    const int n = 16 * j + 4 * grp;
    if (live && n < N) {
      const half4 b4 = __builtin_bit_cast(half4, bb[i]);
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lora = static_cast<float>(h16(static_cast<float>(h16(o[e])) * scaling));
        r[e] = static_cast<float>(b4[e]) + lora;
      }
      *reinterpret_cast<float4*>(out + static_cast<int64_t>(t) * N + n) =
          make_float4(r[0], r[1], r[2], r[3]);
    }
  }
}

// Backward-1. ga[rows x 16] = g . fp16(B), step s (outputs 32 s .. 32 s + 31) on wavefront s % 8;
// lane l brings row l % 16's gradient at outputs 32 s + 4 g .. +3 and 32 s + 16 + 4 g .. +3
// (writing gbase and g there) and fp16(B)[those 8 outputs][rank l % 16]. SN bounds the steps per
// wavefront.
struct Bwd1Job {
  const float* grad;
  const float* B;
  _Float16* gbase;
  _Float16* g16;
  _Float16* ga16;
  int N;
};
struct Bwd1Jobs {
  Bwd1Job j[kMaxJobs];
};

template <int SN>
__global__ __launch_bounds__(kThreads) void lora_fused_bwd1_kernel(Bwd1Jobs jobs, int T,
                                                                   int rows, float scaling) {
  const Bwd1Job jb = jobs.j[blockIdx.y];
  const float* __restrict__ grad = jb.grad;
  const float* __restrict__ B = jb.B;
  _Float16* __restrict__ gbase = jb.gbase;
  _Float16* __restrict__ g16 = jb.g16;
  _Float16* __restrict__ ga16 = jb.ga16;
  const int N = jb.N;
  __shared__ acc4 red[kWaves][cm::kWave];
  const int lane = threadIdx.x % cm::kWave, wave = wave_index();
  const int r16 = lane % 16, grp = lane / 16;
  const int t = blockIdx.x * rows + r16;
  const bool live = r16 < rows && t < T;
  const int steps = (N + 31) / 32;
  // lanes past the tile repeat its last row (the same cache lines, no extra traffic)
  const int64_t tc = min(blockIdx.x * rows + min(r16, rows - 1), T - 1);
  float4 gv[SN][2];
  float bw[SN][8];
#pragma unroll
  for (int i = 0; i < SN; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int n = min(32 * (wave + kWaves * i) + 16 * h + 4 * grp, N - 4);
      gv[i][h] = *reinterpret_cast<const float4*>(grad + tc * N + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) bw[i][4 * h + e] = B[static_cast<int64_t>(n + e) * kR + r16];
    }
  }
  acc4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < SN; ++i) {
    const int s = wave + kWaves * i;
    if (s >= steps) break;
    const float gs[8] = {gv[i][0].x, gv[i][0].y, gv[i][0].z, gv[i][0].w,
                         gv[i][1].x, gv[i][1].y, gv[i][1].z, gv[i][1].w};
    const bool in0 = 32 * s + 4 * grp < N, in1 = 32 * s + 16 + 4 * grp < N;
    half8 gb, g, gm, bh;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = e < 4 ? in0 : in1;
      gb[e] = h16(gs[e]);
      g[e] = h16(static_cast<float>(gb[e]) * scaling);
      gm[e] = in ? g[e] : static_cast<_Float16>(0.0f);
      bh[e] = h16(in ? bw[i][e] : 0.0f);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int n = 32 * s + 16 * h + 4 * grp;
      if (live && n < N) {
        const int64_t at = static_cast<int64_t>(t) * N + n;
        *reinterpret_cast<half4*>(gbase + at) = half4{gb[4 * h], gb[4 * h + 1], gb[4 * h + 2], gb[4 * h + 3]};
        *reinterpret_cast<half4*>(g16 + at) = half4{g[4 * h], g[4 * h + 1], g[4 * h + 2], g[4 * h + 3]};
      }
    }
    acc = mfma_k32(gm, bh, acc);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    // lane l holds rank l % 16 of rows 4 (l / 16) .. +3
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * grp + e;
      const int tm = blockIdx.x * rows + m;
      if (m < rows && tm < T)
        ga16[static_cast<int64_t>(tm) * kR + r16] = h16(sum_waves(red, lane, e));
    }
  }
}

// Backward-2 needs no sum across lanes (each input's gxd is a rank-16 sum): lane c of the
// workgroup owns inputs 4 c .. 4 c + 3 of R token rows. Its 16 columns of fp16(A) (one 16-byte
// read per rank, contiguous across the lanes) serve all R rows, and every row's dxb (or dx), x16
// and mask nibble are loaded at once, so a workgroup waits for memory once. gxd sums the 16
// rank products in rank order. MODE is 0 without dx, 1 for dx = dxb + term, 2 for dx += term (a
// compile-time choice: a branch on it between the loads would make the compiler wait for each
// row's loads in turn).
template <int R, int MODE>
__global__ __launch_bounds__(kMaxK / 4) void lora_fused_bwd2_kernel(
    const _Float16* __restrict__ dxb, const _Float16* __restrict__ ga16,
    const float* __restrict__ A, const _Float16* __restrict__ x16,
    const uint8_t* __restrict__ bits, float* __restrict__ dx, _Float16* __restrict__ xd16,
    int T, int K, float scale_p) {
  __shared__ half8 s_g[R][2];  // ga of the workgroup's rows
  const int c = threadIdx.x, K4 = K / 4, K8 = K / 8, t0 = blockIdx.x * R;
  const bool kok = c < K4;
  const int cc = kok ? c : K4 - 1;  // clamped column quad
  uint4 prior[R];  // the 4 fp16 of dxb in .x/.y, or the 4 fp32 of dx as it is (accumulating)
  uint2 xq[R];
  uint32_t mb[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t tc = min(t0 + i, T - 1);
    const int64_t at = tc * K + 4 * cc;
    if constexpr (MODE == 1) {
      const uint2 d = *reinterpret_cast<const uint2*>(dxb + at);
      prior[i] = make_uint4(d.x, d.y, 0u, 0u);
    } else if constexpr (MODE == 2) {
      prior[i] = *reinterpret_cast<const uint4*>(dx + at);
    } else {
      prior[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    xq[i] = *reinterpret_cast<const uint2*>(x16 + at);
    mb[i] = bits[tc * K8 + cc / 2];
  }
  float4 ac[kR];  // fp32 A[r][4 c .. 4 c + 3], then its fp16 values
#pragma unroll
  for (int r = 0; r < kR; ++r)
    ac[r] = *reinterpret_cast<const float4*>(A + static_cast<int64_t>(r) * K + 4 * cc);
  if (threadIdx.x < 2 * R) {
    const int i = threadIdx.x / 2, h = threadIdx.x % 2;
    s_g[i][h] = *reinterpret_cast<const half8*>(
        ga16 + static_cast<int64_t>(min(t0 + i, T - 1)) * kR + 8 * h);
  }
  __syncthreads();
  if (!kok) return;  // no barrier below
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    ac[r].x = static_cast<float>(h16(ac[r].x));
    ac[r].y = static_cast<float>(h16(ac[r].y));
    ac[r].z = static_cast<float>(h16(ac[r].z));
    ac[r].w = static_cast<float>(h16(ac[r].w));
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (t0 + i >= T) break;
    const half8 g0 = s_g[i][0], g1 = s_g[i][1];
    float gx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const float g = static_cast<float>(r < 8 ? g0[r] : g1[r - 8]);
      gx[0] += g * ac[r].x;
      gx[1] += g * ac[r].y;
      gx[2] += g * ac[r].z;
      gx[3] += g * ac[r].w;
    }
    const uint32_t nib = (mb[i] >> (4 * (c & 1))) & 0xfu;
    const half4 db = __builtin_bit_cast(half4, make_uint2(prior[i].x, prior[i].y));
    const half4 xv = __builtin_bit_cast(half4, xq[i]);
    const uint32_t dold[4] = {prior[i].x, prior[i].y, prior[i].z, prior[i].w};
    float o[4];
    half4 xo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool kept = (nib >> e) & 1u;
      const float gl = kept ? static_cast<float>(h16(gx[e])) * scale_p : 0.0f;
      o[e] = (MODE == 1 ? static_cast<float>(db[e]) : __uint_as_float(dold[e])) + gl;
      xo[e] = h16(kept ? static_cast<float>(xv[e]) * scale_p : 0.0f);
    }
    const int64_t at = static_cast<int64_t>(t0 + i) * K + 4 * c;
    if constexpr (MODE != 0)
      *reinterpret_cast<float4*>(dx + at) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<half4*>(xd16 + at) = xo;
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Per-wavefront bounds: steps of 32 (tiles of 16) over `len` split 8 ways, rounded up to the
// instantiated sizes.
int steps_bound(int len) {
  const int per = ((len + 31) / 32 + kWaves - 1) / kWaves;
  return per <= 2 ? 2 : per <= 4 ? 4 : per <= 6 ? 6 : 8;
}
int tiles_bound(int len) {
  const int per = ((len + 15) / 16 + kWaves - 1) / kWaves;
  return per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : per <= 12 ? 12 : 16;
}

// Token rows per workgroup of the column-quad kernels: the most (of 1, 2, 4, 8, 16) that still
// gives the CUs a workgroup each.
int quad_rows(int64_t T) {
  int r = 16;
  while (r > 1 && (T + r - 1) / r < kCUs) r /= 2;
  return r;
}

// Token rows per tile: 16, or fewer when 16-row tiles would leave CUs idle.
int tile_rows(int64_t T) {
  const int64_t r = (T + kCUs - 1) / kCUs;
  return static_cast<int>(std::min<int64_t>(kTileRows, std::max<int64_t>(1, r)));
}
dim3 tile_grid(int64_t T, int rows) { return dim3(static_cast<unsigned>((T + rows - 1) / rows)); }

}  // namespace

#define CM_LORA_SK_SWITCH(v, SK, ...)                     \
  switch (v) {                                            \
    case 2: { constexpr int SK = 2; __VA_ARGS__; break; } \
    case 4: { constexpr int SK = 4; __VA_ARGS__; break; } \
    case 6: { constexpr int SK = 6; __VA_ARGS__; break; } \
    default: { constexpr int SK = 8; __VA_ARGS__; break; } \
  }
#define CM_LORA_SN_SWITCH(v, SN, ...)                       \
  switch (v) {                                              \
    case 2: { constexpr int SN = 2; __VA_ARGS__; break; }   \
    case 4: { constexpr int SN = 4; __VA_ARGS__; break; }   \
    case 8: { constexpr int SN = 8; __VA_ARGS__; break; }   \
    case 12: { constexpr int SN = 12; __VA_ARGS__; break; } \
    default: { constexpr int SN = 16; __VA_ARGS__; break; } \
  }

#define CM_LORA_J_SWITCH(v, J, ...)                        \
  switch (v) {                                             \
    case 1: { constexpr int J = 1; __VA_ARGS__; break; }   \
    case 2: { constexpr int J = 2; __VA_ARGS__; break; }   \
    case 4: { constexpr int J = 4; __VA_ARGS__; break; }   \
    case 8: { constexpr int J = 8; __VA_ARGS__; break; }   \
    default: { constexpr int J = 16; __VA_ARGS__; break; } \
  }

namespace {

// The checks of one adapter of cm_lora_fused_fwd / _fwd_multi.
bool fwd_job_ok(const float* x, const uint8_t* keep, const float* weight_a, const float* weight_b,
                const void* base16, const float* out, const uint8_t* bits, const void* a16,
                int K, int N) {
  return N > 0 && N % 8 == 0 && N <= kMaxN && x && keep && weight_a && weight_b && base16 &&
         out && bits && a16 && aligned(x, 16) && aligned(keep, 8) && aligned(weight_a, 16) &&
         aligned(weight_b, 16) && aligned(base16, 8) && aligned(out, 16) && aligned(a16, 8) &&
         K % 8 == 0;
}

int launch_fwd(const float* x, const FwdJobs& jobs, int n_jobs, int max_n, int64_t T, int K,
               float scale_p, float scaling, hipStream_t s) {
  const int rows = tile_rows(T);
  dim3 grid = tile_grid(T, rows);
  grid.y = n_jobs;
  CM_LORA_SK_SWITCH(steps_bound(K), SK, CM_LORA_SN_SWITCH(tiles_bound(max_n), SN, {
    hipLaunchKernelGGL((lora_fused_fwd_kernel<SK, SN>), grid, dim3(kThreads), 0, s, x, jobs,
                       static_cast<int>(T), K, rows, scale_p, scaling);
  }));
  return cm::launch_status();
}

bool bwd1_job_ok(const float* grad, const float* weight_b, const void* gbase16, const void* g16,
                 const void* ga16, int N) {
  return N > 0 && N % 8 == 0 && N <= kMaxN && grad && weight_b && gbase16 && g16 && ga16 &&
         aligned(grad, 16) && aligned(weight_b, 4) && aligned(gbase16, 8) && aligned(g16, 8) &&
         aligned(ga16, 2);
}

int launch_bwd1(const Bwd1Jobs& jobs, int n_jobs, int max_n, int64_t T, float scaling,
                hipStream_t s) {
  const int rows = tile_rows(T);
  dim3 grid = tile_grid(T, rows);
  grid.y = n_jobs;
  CM_LORA_SK_SWITCH(steps_bound(max_n), SN, {
    hipLaunchKernelGGL(lora_fused_bwd1_kernel<SN>, grid, dim3(kThreads), 0, s, jobs,
                       static_cast<int>(T), rows, scaling);
  });
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_lora_fused_fwd(const float* x, const uint8_t* keep, const float* weight_a,
                                 const float* weight_b, const void* base16, float* out,
                                 uint8_t* bits, void* a16, int64_t T, int K, int N, int rank,
                                 float scale_p, float scaling, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && K > 0 && N > 0);
  CM_CHECK_ARG(K % 8 == 0 && N % 8 == 0 && K <= kMaxK && N <= kMaxN);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  CM_CHECK_ARG(fwd_job_ok(x, keep, weight_a, weight_b, base16, out, bits, a16, K, N));
  FwdJobs jobs{};
  jobs.j[0] = FwdJob{keep, weight_a, weight_b, static_cast<const _Float16*>(base16), out, bits,
                     static_cast<_Float16*>(a16), N};
  return launch_fwd(x, jobs, 1, N, T, K, scale_p, scaling, static_cast<hipStream_t>(stream));
}

extern "C" int cm_lora_fused_fwd_multi(const float* x, int64_t T, int K, int rank, float scale_p,
                                       float scaling, int n_jobs, const uint8_t* const* keep,
                                       const float* const* weight_a,
                                       const float* const* weight_b, const void* const* base16,
                                       float* const* out, uint8_t* const* bits,
                                       void* const* a16, const int* N, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && K > 0 && K % 8 == 0 && K <= kMaxK);
  CM_CHECK_ARG(n_jobs >= 1 && n_jobs <= kMaxJobs);
  CM_CHECK_ARG(keep && weight_a && weight_b && base16 && out && bits && a16 && N);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  FwdJobs jobs{};
  int max_n = 0;
  for (int i = 0; i < n_jobs; ++i) {
    CM_CHECK_ARG(fwd_job_ok(x, keep[i], weight_a[i], weight_b[i], base16[i], out[i], bits[i],
                            a16[i], K, N[i]));
    jobs.j[i] = FwdJob{keep[i], weight_a[i], weight_b[i],
                       static_cast<const _Float16*>(base16[i]), out[i], bits[i],
                       static_cast<_Float16*>(a16[i]), N[i]};
    max_n = std::max(max_n, N[i]);
  }
  return launch_fwd(x, jobs, n_jobs, max_n, T, K, scale_p, scaling,
                    static_cast<hipStream_t>(stream));
}

extern "C" int cm_lora_fused_bwd1(const float* grad, const float* weight_b, void* gbase16,
                                  void* g16, void* ga16, int64_t T, int N, int rank,
                                  float scaling, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && N > 0 && N % 8 == 0 && N <= kMaxN);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  CM_CHECK_ARG(bwd1_job_ok(grad, weight_b, gbase16, g16, ga16, N));
  Bwd1Jobs jobs{};
  jobs.j[0] = Bwd1Job{grad, weight_b, static_cast<_Float16*>(gbase16),
                      static_cast<_Float16*>(g16), static_cast<_Float16*>(ga16), N};
  return launch_bwd1(jobs, 1, N, T, scaling, static_cast<hipStream_t>(stream));
}

extern "C" int cm_lora_fused_bwd1_multi(int64_t T, int rank, float scaling, int n_jobs,
                                        const float* const* grad, const float* const* weight_b,
                                        void* const* gbase16, void* const* g16,
                                        void* const* ga16, const int* N, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && n_jobs >= 1 && n_jobs <= kMaxJobs);
  CM_CHECK_ARG(grad && weight_b && gbase16 && g16 && ga16 && N);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  Bwd1Jobs jobs{};
  int max_n = 0;
  for (int i = 0; i < n_jobs; ++i) {
    CM_CHECK_ARG(bwd1_job_ok(grad[i], weight_b[i], gbase16[i], g16[i], ga16[i], N[i]));
    jobs.j[i] = Bwd1Job{grad[i], weight_b[i], static_cast<_Float16*>(gbase16[i]),
                        static_cast<_Float16*>(g16[i]), static_cast<_Float16*>(ga16[i]), N[i]};
    max_n = std::max(max_n, N[i]);
  }
  return launch_bwd1(jobs, n_jobs, max_n, T, scaling, static_cast<hipStream_t>(stream));
}

extern "C" int cm_lora_fused_bwd2(const void* dxb16, const void* ga16, const float* weight_a,
                                  const void* x16, const uint8_t* bits, float* dx, void* xd16,
                                  int64_t T, int K, int rank, float scale_p, void* stream) {
  CM_CHECK_ARG(rank == kR && T >= 0 && K > 0 && K % 8 == 0 && K <= kMaxK);
  if (T == 0) return 0;
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  CM_CHECK_ARG(ga16 && weight_a && x16 && bits && xd16);
  CM_CHECK_ARG((!dx || ((!dxb16 || aligned(dxb16, 8)) && aligned(dx, 16))) && aligned(ga16, 16) &&
               aligned(weight_a, 16) && aligned(x16, 8) && aligned(xd16, 8));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int mode = !dx ? 0 : dxb16 ? 1 : 2;
  const int R = quad_rows(T);
  const dim3 grid(static_cast<unsigned>((T + R - 1) / R)), block((K / 4 + 63) / 64 * 64);
  CM_LORA_J_SWITCH(R, RR, {
    const auto kernel = mode == 0   ? lora_fused_bwd2_kernel<RR, 0>
                        : mode == 1 ? lora_fused_bwd2_kernel<RR, 1>
                                    : lora_fused_bwd2_kernel<RR, 2>;
    hipLaunchKernelGGL(kernel, grid, block, 0, s, static_cast<const _Float16*>(dxb16),
                       static_cast<const _Float16*>(ga16), weight_a,
                       static_cast<const _Float16*>(x16), bits, dx, static_cast<_Float16*>(xd16),
                       static_cast<int>(T), K, scale_p);
  });
  return cm::launch_status();
}

// ---------------------------------------------------------------------------------------------
// The adapters' weight gradients, several at once: for each job, out = sum over the T token
// rows of outer(W[t], R[t]), W [T, D] fp16 (row stride ldw), R [T, 16] fp16, in fp32:
//   lora_A's gradient  ga16^T xd16 : W = xd16 (D = K), R = ga16, out [16, K]  (rank-major)
//   lora_B's gradient  g16^T a16   : W = g16  (D = N), R = a16,  out [N, 16]  (column-major)
// The reference computes each as a GEMM over the tokens (solution/lora.py:96-107). Here one
// workgroup takes 32 columns of one job over all the tokens: a product out[16 ranks x 16 columns]
// is v_mfma_f32_16x16x32_f16 steps of 32 tokens with the ranks as the left operand (R^T) and the
// columns as the right one (W), the tokens being the contraction, so that no lane needs another
// lane's data. Lane l supplies rank l % 16 and the column pair col0 + 2 (l % 16) .. +1 (the even
// column to the first tile, the odd one to the second) over the 8 tokens 8 (l / 16) .. +7 of a
// step: 2- and 4-byte loads whose 16 lanes of a group read 32 or 64 contiguous bytes of one token
// row (a load instruction's cost is per lane, not per byte, at these widths). The 8
// wavefronts take the steps in turn (step s on wavefront s % 8), each loading several steps
// before it multiplies them, and their 16 x 16 sums are added through the LDS in a fixed order:
// one launch, no workspace, and the same inputs give the same bits. The products of two fp16
// values are exact in fp32, so the sums differ from a GEMM's only in their order.
namespace {

constexpr int kWgJobs = 4;
constexpr int kWgCols = 32;    // columns of W per workgroup: two 16-column MFMA tiles
constexpr int kWgWaves = 8;    // wavefronts per workgroup, splitting the tokens
constexpr int kWgBatch = 2;    // 32-token steps a wavefront loads before it multiplies them
                               // (2 to 5 measured: 2 and 3 fastest at 1276 and 5000 tokens)

struct WgJob {
  const _Float16* w;
  int64_t ldw;
  const _Float16* r;
  float* out;
  int d;        // columns of W
  int d_major;  // out[d][r] (else out[r][d])
};
struct WgJobs {
  WgJob j[kWgJobs];
};

__global__ __launch_bounds__(kWgWaves * cm::kWave) void lora_wgrad_kernel(WgJobs jobs,
                                                                           int64_t T) {
  __shared__ acc4 s_part[kWgWaves][2][cm::kWave];
  const WgJob jb = jobs.j[blockIdx.y];
  const int col0 = blockIdx.x * kWgCols;
  if (col0 >= jb.d) return;  // this job has fewer columns (uniform per workgroup)
  const int lane = threadIdx.x % cm::kWave, wave = wave_index();
  const int c16 = lane % 16, grp = lane / 16;
  // the lane's column pair, clamped into the row (D is a multiple of 8, so a pair is whole;
  // columns past D are not stored)
  const int dc = min(col0 + 2 * c16, jb.d - 2);
  const int64_t steps = (T + 31) / 32;
  acc4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  for (int64_t s0 = wave; s0 < steps; s0 += kWgWaves * kWgBatch) {
    _Float16 rv[kWgBatch][8];
    uint32_t wv[kWgBatch][8];
    // every load first (rows past T clamped to T - 1 and their values zeroed after the loads)
#pragma unroll
    for (int b = 0; b < kWgBatch; ++b) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t t = min((s0 + kWgWaves * b) * 32 + 8 * grp + e, T - 1);
        rv[b][e] = jb.r[t * kR + c16];
        wv[b][e] = *reinterpret_cast<const uint32_t*>(jb.w + t * jb.ldw + dc);
      }
    }
#pragma unroll
    for (int b = 0; b < kWgBatch; ++b) {
      const int64_t s = s0 + kWgWaves * b;
      if (s >= steps) break;
      half8 ra, wa, wb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool in = s * 32 + 8 * grp + e < T;
        const _Float16 lo = __builtin_bit_cast(_Float16, static_cast<uint16_t>(wv[b][e]));
        const _Float16 hi = __builtin_bit_cast(_Float16, static_cast<uint16_t>(wv[b][e] >> 16));
        ra[e] = in ? rv[b][e] : static_cast<_Float16>(0.0f);
        wa[e] = in ? lo : static_cast<_Float16>(0.0f);
        wb[e] = in ? hi : static_cast<_Float16>(0.0f);
      }
      acc0 = mfma_k32(ra, wa, acc0);
      acc1 = mfma_k32(ra, wb, acc1);
    }
  }
  s_part[wave][0][lane] = acc0;
  s_part[wave][1][lane] = acc1;
  __syncthreads();
  if (wave >= 2) return;
  // wavefront v adds tile v over the 8 wavefronts; lane l holds ranks 4 (l / 16) .. +3 of
  // column col0 + 2 (l % 16) + v
  const int d = col0 + 2 * c16 + wave;
  acc4 sum;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v[kWgWaves];
#pragma unroll
    for (int w = 0; w < kWgWaves; ++w) v[w] = s_part[w][wave][lane][i];
    sum[i] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  }
  if (d >= jb.d) return;
  if (jb.d_major) {
    *reinterpret_cast<float4*>(jb.out + static_cast<int64_t>(d) * kR + 4 * grp) =
        make_float4(sum[0], sum[1], sum[2], sum[3]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) jb.out[static_cast<int64_t>(4 * grp + i) * jb.d + d] = sum[i];
  }
}

}  // namespace

extern "C" int64_t cm_lora_weight_grads_workspace_bytes(int64_t T, int max_d, int n_jobs) {
  if (T < 0 || max_d <= 0 || n_jobs < 1 || n_jobs > kWgJobs) return -1;
  return 0;  // one launch, its sums in the LDS
}

extern "C" int cm_lora_weight_grads(const void* const* w, const int64_t* ldw, const int* d,
                                    const void* const* r, float* const* out,
                                    const int* d_major, int n_jobs, int64_t T, int rank,
                                    void* workspace, int64_t ws_bytes, void* stream) {
  (void)workspace;
  (void)ws_bytes;
  CM_CHECK_ARG(rank == kR && n_jobs >= 1 && n_jobs <= kWgJobs && T >= 0);
  CM_CHECK_ARG(w && ldw && d && r && out && d_major);
  CM_CHECK_ARG(T <= 0x7fffffff / 2);
  WgJobs jobs{};
  int max_d = 0;
  for (int q = 0; q < n_jobs; ++q) {
    // with no tokens w and r are not read (empty arrays may have no address)
    CM_CHECK_ARG((T == 0 || (w[q] && r[q])) && out[q] && d[q] > 0 && d[q] % 8 == 0 &&
                 ldw[q] >= d[q] && ldw[q] % 2 == 0);
    CM_CHECK_ARG((reinterpret_cast<uintptr_t>(w[q]) & 3) == 0 && aligned(r[q], 16) &&
                 aligned(out[q], d_major[q] ? 16 : 4));
    jobs.j[q] = WgJob{static_cast<const _Float16*>(w[q]), ldw[q],
                      static_cast<const _Float16*>(r[q]), out[q], d[q], d_major[q] ? 1 : 0};
    max_d = std::max(max_d, d[q]);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(lora_wgrad_kernel, dim3((max_d + kWgCols - 1) / kWgCols, n_jobs),
                     dim3(kWgWaves * cm::kWave), 0, s, jobs, T);
  return cm::launch_status();
}
