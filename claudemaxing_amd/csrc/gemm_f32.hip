// Split-K fp16 GEMM with an fp32 result, for the products of the training step whose output is
// small next to their contraction (gfx950): C[m][n] = sum_k A[m][k] B[n][k] (+ the same over a
// second pair A2, B2 with its own K), A [M, K] and B [N, K] fp16 row-major (both read along k).
//
// At 1276 tokens the MLP's down projection (K = 8960 -> N = 1536) and its input gradient
// (K = 2 x 8960 -> N = 1536) have 40 output tiles of 256 x 192: far fewer than the 256 CUs, each
// a long contraction, which hipBLASLt's solutions for these shapes run at ~500-570 TFLOP/s. Here
// the contraction is cut into K-slices of whole 64-column stages, each slice within one pair,
// so tiles x slices fills the chip; each workgroup runs the gemm_lds main loop (direct
// global -> LDS loads, v_mfma_f32_32x32x16_f16) over its slice and writes its fp32 partial tile
// to a workspace slice, and a second kernel adds the slices in slice order (deterministic: the
// same inputs give the same bits). The workspace is S x M x N fp32.
//
// B may also be given k-major (cm_gemm_f32_kb: B[n][k] at b[k * ldb + n], a weight as stored
// for the input gradient dX = G W): its LDS tiles are then read with transposing fragment reads
// that hand each lane the same (n, k) elements as the row-major path, so the two give the same
// bits for the same values.
#include "gemm_lds.h"

namespace {

using cm::gemm::floatx16;
using cm::gemm::KMajor;
using cm::gemm::RowMajor;

constexpr int kBM = 256, kBN = 192, kWM = 4, kWN = 2, kBK = 64, kStages = 2;
constexpr int kThreads = kWM * kWN * cm::kWave;
constexpr int kMaxSlices = 16;
constexpr int kCUs = 256;

// The fp32 partial tile of one K-slice, rows past M and columns past N dropped.
struct EpiSlice {
  float* out;  // [M, N] slice of the workspace
  int M, N;
  template <int TM, int TN>
  __device__ __forceinline__ void prepare(int, int, int) {}
  template <int TM, int TN>
  __device__ __forceinline__ void start(floatx16 (&acc)[TM][TN], int mb, int nb, int lane) {
    cm::gemm::ZeroStart::start<TM, TN>(acc, mb, nb, lane);
  }
  template <int TM, int TN>
  __device__ __forceinline__ void started(floatx16 (&)[TM][TN]) {}
  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb, int lane,
                                        uint4*) const {
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = mb + mt * 32 + (r / 4) * 8 + (lane / 32) * 4 + (r % 4);
        if (row >= M) continue;
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          const int col = nb + nt * 32 + lane % 32;
          if (col < N) out[static_cast<int64_t>(row) * N + col] = acc[mt][nt][r];
        }
      }
  }
};

struct Pairs {
  RowMajor a[2], b[2];
  KMajor bk[2];     // B of each pair when the kernel takes it k-major
  int slices0;      // slices of pair 0; the rest belong to pair 1
  int k_slice[2];   // columns per slice of each pair (a multiple of 64)
};

template <bool KB>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_kernel(Pairs p, int remap, float* ws,
                                                               int M, int N) {
  __shared__ uint4 lds[kStages * (kBM + kBN) * (kBK / 8)];
  int tm, tn, s;
  cm::gemm::tile_of_block_2d((N + kBN - 1) / kBN, remap, tm, tn, s);
  const int q = s < p.slices0 ? 0 : 1, sq = q ? s - p.slices0 : s;
  const int k_begin = sq * p.k_slice[q];
  // an empty slice still writes its (zero) partial tile, which the sum then reads
  const int k_end = max(k_begin, min(p.a[q].k_len, k_begin + p.k_slice[q]));
  EpiSlice epi{ws + static_cast<int64_t>(s) * M * N, M, N};
  if constexpr (KB) {
    if (q == 0) {
      cm::gemm::gemm_lds<kBM, kBN, kWM, kWN, kBK, kStages>(p.a[0], p.bk[0], k_begin, k_end, tm,
                                                           tn, epi, lds);
    } else {
      cm::gemm::gemm_lds<kBM, kBN, kWM, kWN, kBK, kStages>(p.a[1], p.bk[1], k_begin, k_end, tm,
                                                           tn, epi, lds);
    }
  } else {
    if (q == 0) {
      cm::gemm::gemm_lds<kBM, kBN, kWM, kWN, kBK, kStages>(p.a[0], p.b[0], k_begin, k_end, tm,
                                                           tn, epi, lds);
    } else {
      cm::gemm::gemm_lds<kBM, kBN, kWM, kWN, kBK, kStages>(p.a[1], p.b[1], k_begin, k_end, tm,
                                                           tn, epi, lds);
    }
  }
}

// out = sum over the S slices in slice order, 4 values per lane; with `residual`, out = residual
// + that sum (the residual add of the layer the product ends, one more fp32 rounding).
__global__ __launch_bounds__(256) void gemm_f32_sum(const float4* __restrict__ ws, int S,
                                                    int64_t n4, float4* __restrict__ out,
                                                    const float4* __restrict__ residual) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  // the slices are loaded 8 at a time before they are added in slice order (a runtime-length
  // loop of load-then-add would wait for each load in turn)
  float4 a = ws[i];
  for (int s0 = 1; s0 < S; s0 += 8) {
    float4 b[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (s0 + k < S) b[k] = ws[(s0 + k) * n4 + i];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (s0 + k < S) {
        a.x += b[k].x; a.y += b[k].y; a.z += b[k].z; a.w += b[k].w;
      }
  }
  if (residual != nullptr) {
    const float4 r = residual[i];
    a.x = r.x + a.x; a.y = r.y + a.y; a.z = r.z + a.z; a.w = r.w + a.w;
  }
  out[i] = a;
}

struct Plan {
  int slices[2];
  int k_slice[2];
  int total() const { return slices[0] + slices[1]; }
};

// Slices per pair in proportion to its K, so that tiles x slices is one round of workgroups
// (one per CU: the LDS ring takes 112 KiB), in whole 64-column stages, at most 16 slices. At
// 40 tiles: 6 slices, 240 workgroups (10 slices in 1.6 rounds measured slower).
Plan plan_for(int M, int N, int K0, int K1) {
  const int tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int want = std::max(1, std::min(kMaxSlices, kCUs / tiles));
  Plan pl{};
  const int64_t k_all = static_cast<int64_t>(K0) + K1;
  const int ks[2] = {K0, K1};
  for (int q = 0; q < 2; ++q) {
    if (ks[q] == 0) {
      pl.slices[q] = 0;
      pl.k_slice[q] = kBK;
      continue;
    }
    int sq = static_cast<int>(std::max<int64_t>(1, (want * static_cast<int64_t>(ks[q]) + k_all / 2) / k_all));
    const int stages = (ks[q] + kBK - 1) / kBK;
    sq = std::min(sq, stages);
    pl.k_slice[q] = (stages + sq - 1) / sq * kBK;
    pl.slices[q] = (ks[q] + pl.k_slice[q] - 1) / pl.k_slice[q];
  }
  return pl;
}

bool shape_ok(int M, int N, int K0, int K1) {
  return M >= 0 && N >= 0 && K0 > 0 && K1 >= 0 && K0 % 8 == 0 && K1 % 8 == 0;
}

}  // namespace

extern "C" int64_t cm_gemm_f32_workspace_bytes(int M, int N, int K0, int K1) {
  if (!shape_ok(M, N, K0, K1)) return -1;
  if (M == 0 || N == 0) return 0;
  return static_cast<int64_t>(plan_for(M, N, K0, K1).total()) * M * N * 4;
}

namespace {

int gemm_f32_impl(const void* a0, int64_t lda0, const void* b0, int64_t ldb0, int K0,
                  const void* a1, int64_t lda1, const void* b1, int64_t ldb1, int K1, int M,
                  int N, const float* residual, float* out, void* workspace, int64_t ws_bytes,
                  void* stream, bool b_kmajor = false) {
  CM_CHECK_ARG(shape_ok(M, N, K0, K1));
  if (M == 0 || N == 0) return 0;
  CM_CHECK_ARG(a0 && b0 && out && workspace && (K1 == 0 || (a1 && b1)));
  // B's rows: K of them of N values when k-major (N a multiple of 8: whole 16-byte chunks), else
  // N rows of K
  const int64_t b_row = b_kmajor ? N : 0;
  CM_CHECK_ARG(!b_kmajor || N % 8 == 0);
  CM_CHECK_ARG(lda0 >= K0 && lda0 % 8 == 0 && ldb0 % 8 == 0 && ldb0 >= (b_kmajor ? b_row : K0));
  CM_CHECK_ARG(K1 == 0 || (lda1 >= K1 && lda1 % 8 == 0 && ldb1 % 8 == 0 &&
                           ldb1 >= (b_kmajor ? b_row : K1)));
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  CM_CHECK_ARG(al16(a0) && al16(b0) && al16(out) && al16(workspace) &&
               (K1 == 0 || (al16(a1) && al16(b1))) && (!residual || al16(residual)));
  CM_CHECK_ARG(static_cast<int64_t>(M) * N % 4 == 0);
  const Plan pl = plan_for(M, N, K0, K1);
  CM_CHECK_ARG(ws_bytes >= static_cast<int64_t>(pl.total()) * M * N * 4);
  Pairs p{};
  p.a[0] = RowMajor{static_cast<const _Float16*>(a0), lda0, M, K0};
  p.b[0] = RowMajor{static_cast<const _Float16*>(b0), ldb0, N, K0};
  p.a[1] = K1 ? RowMajor{static_cast<const _Float16*>(a1), lda1, M, K1} : p.a[0];
  p.b[1] = K1 ? RowMajor{static_cast<const _Float16*>(b1), ldb1, N, K1} : p.b[0];
  p.bk[0] = KMajor{static_cast<const _Float16*>(b0), ldb0, N, K0};
  p.bk[1] = K1 ? KMajor{static_cast<const _Float16*>(b1), ldb1, N, K1} : p.bk[0];
  p.slices0 = pl.slices[0];
  p.k_slice[0] = pl.k_slice[0];
  p.k_slice[1] = pl.k_slice[1];
  const int tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int remap = (tiles * pl.total()) % 8 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  if (b_kmajor) {
    hipLaunchKernelGGL(gemm_f32_kernel<true>, dim3(tiles, pl.total()), dim3(kThreads), 0, s, p,
                       remap, ws, M, N);
  } else {
    hipLaunchKernelGGL(gemm_f32_kernel<false>, dim3(tiles, pl.total()), dim3(kThreads), 0, s, p,
                       remap, ws, M, N);
  }
  const int64_t n4 = static_cast<int64_t>(M) * N / 4;
  hipLaunchKernelGGL(gemm_f32_sum, dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<const float4*>(ws), pl.total(), n4,
                     reinterpret_cast<float4*>(out), reinterpret_cast<const float4*>(residual));
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_gemm_f32(const void* a0, int64_t lda0, const void* b0, int64_t ldb0, int K0,
                           const void* a1, int64_t lda1, const void* b1, int64_t ldb1, int K1,
                           int M, int N, float* out, void* workspace, int64_t ws_bytes,
                           void* stream) {
  return gemm_f32_impl(a0, lda0, b0, ldb0, K0, a1, lda1, b1, ldb1, K1, M, N, nullptr, out,
                       workspace, ws_bytes, stream);
}

extern "C" int cm_gemm_f32_add(const void* a0, int64_t lda0, const void* b0, int64_t ldb0,
                               int K0, const void* a1, int64_t lda1, const void* b1,
                               int64_t ldb1, int K1, int M, int N, const float* residual,
                               float* out, void* workspace, int64_t ws_bytes, void* stream) {
  CM_CHECK_ARG(M == 0 || N == 0 || residual != nullptr);
  return gemm_f32_impl(a0, lda0, b0, ldb0, K0, a1, lda1, b1, ldb1, K1, M, N, residual, out,
                       workspace, ws_bytes, stream);
}

extern "C" int cm_gemm_f32_kb(const void* a0, int64_t lda0, const void* b0, int64_t ldb0, int K0,
                              const void* a1, int64_t lda1, const void* b1, int64_t ldb1, int K1,
                              int M, int N, float* out, void* workspace, int64_t ws_bytes,
                              void* stream) {
  return gemm_f32_impl(a0, lda0, b0, ldb0, K0, a1, lda1, b1, ldb1, K1, M, N, nullptr, out,
                       workspace, ws_bytes, stream, true);
}
