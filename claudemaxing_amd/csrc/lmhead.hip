// Fused LM head + cross-entropy with per-row loss, entropy, accuracy and the hidden-state
// gradient (gfx950, fp16 MFMA with fp32 accumulation).
//
// Reproduces _FusedHeadLoss of the reference (solution/lm_head_loss.py:192-254: per vocabulary
// chunk torch.mm -> lm_head_vocab_chunk_kernel (108-160) -> torch.mm, then the label fix-up
// 230-236). The vocabulary is walked in chunks of C columns; per chunk four launches run on the
// caller's stream:
//
//   K1 logits   Z^T = W_c H^T on the matrix cores (256 x 256 workgroup tiles of
//               v_mfma_f32_32x32x16_f16, K = hidden in steps of 64 staged through LDS). The
//               epilogue rounds each logit to fp16 (the base path's fp16 logits), stores the fp16
//               chunk row-major [tokens, C] and reduces every token's 128-column groups to
//               partial online-softmax statistics (max, sum e^{z-max}, sum e^{z-max} z, first
//               argmax) straight from the accumulators: a lane holds 64 logits of one token.
//   K2 rows     per token: merge the chunk's partials into the running statistics, record the
//               label logit and the rescale factor e^{lse_before - lse_after}; with a gradient,
//               overwrite the fp16 chunk in place by P = fp16(e^{z - lse_after} * 1024) (zero for
//               unlabelled tokens; the power-of-two scale keeps the small probabilities of a
//               152K vocabulary out of fp16's subnormal range).
//   K3 grad     G = G * factor + P W_c on the matrix cores (128 x 128 tiles; the B operand is the
//               transposed weight chunk, so both operands stream K-contiguous 16-byte rows).
//   K4 final    (after the last chunk) lse, loss, entropy, correct; G = scale (G / 1024 - W_t).
//
// The full [tokens, vocab] logits never exist: one fp16 chunk lives in the workspace, sized so
// that it, the weight chunk and its transpose stay inside the 256 MB Infinity Cache.
//
// Tile loads use 16-byte accesses; LDS rows of 64 fp16 (128 B = 8 chunks of 16 B) are XOR
// swizzled (chunk ^ row % 8) so the per-lane fragment reads of a wavefront hit 32 distinct banks.
#include "common.h"
#include "softmax_state.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;      // 4 wavefronts per workgroup
constexpr int kBK = 64;            // K elements per pipeline stage
constexpr int kRowChunks = kBK / 8;  // 16-byte chunks per LDS tile row
constexpr int kGroup = 128;        // vocabulary columns per partial-statistics group
constexpr float kPScale = 1024.0f;  // P16 = fp16(p * kPScale)
constexpr int kStatThreads = 256;

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// ---------------------------------------------------------------------------------------------
// Tile loader: rows [r0, r0 + ROWS) and columns [k0, k0 + 64) of a row-major fp16 matrix; rows at
// or beyond n_rows and columns at or beyond k_len read as zero.
template <int ROWS>
struct TileLoad {
  static constexpr int kPer = ROWS * kRowChunks / kThreads;
  static_assert(kPer * kThreads == ROWS * kRowChunks, "tile rows must split over the threads");
  uint4 v[kPer];

  __device__ __forceinline__ void load(const _Float16* __restrict__ base, int64_t ld, int r0,
                                       int n_rows, int k0, int k_len) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * kThreads;
      const int row = c / kRowChunks;
      const int k = k0 + (c % kRowChunks) * 8;
      const int r = r0 + row;
      if (r < n_rows && k + 8 <= k_len) {
        v[i] = *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(r) * ld + k);
      } else if (r < n_rows && k < k_len) {
        union {
          uint4 u;
          _Float16 h[8];
        } t;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          t.h[e] = k + e < k_len ? base[static_cast<int64_t>(r) * ld + k + e] : _Float16(0);
        v[i] = t.u;
      } else {
        v[i] = zero4();
      }
    }
  }

  __device__ __forceinline__ void store(uint4* lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * kThreads;
      const int row = c / kRowChunks;
      const int ch = c % kRowChunks;
      lds[row * kRowChunks + (ch ^ (row & 7))] = v[i];
    }
  }
};

__device__ __forceinline__ half8 frag(const uint4* lds, int row, int ch) {
  const uint4 u = lds[row * kRowChunks + (ch ^ (row & 7))];
  return __builtin_bit_cast(half8, u);
}

// ---------------------------------------------------------------------------------------------
// C[m][n] = sum_k A[m][k] B[n][k] for row-major fp16 A [M, K] and B [N, K] (both K-contiguous),
// fp32 accumulation in MFMA 32x32x16 tiles; each wavefront owns a (BM/WM) x (BN/WN) sub-tile and
// hands its accumulators to the epilogue. acc[mt][nt][r] holds
//   row m = m_wave + 32 mt + 8 (r / 4) + 4 (lane / 32) + r % 4,   col n = n_wave + 32 nt + lane % 32.
template <int BM, int BN, int WM, int WN, class Epi>
__global__ __launch_bounds__(kThreads, 1) void gemm_nt(const _Float16* __restrict__ A, int64_t lda,
                                                       int M, const _Float16* __restrict__ B,
                                                       int64_t ldb, int N, int K, int remap,
                                                       Epi epi) {
  static_assert(WM * WN == kThreads / cm::kWave, "four wavefronts");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM * 32 == WTM && TN * 32 == WTN, "wave tiles are multiples of 32");
  __shared__ uint4 lds[2][(BM + BN) * kRowChunks];

  const int tiles_n = (N + BN - 1) / BN;
  int bid = blockIdx.x;
  if (remap) {  // consecutive logical tiles on one XCD (workgroups go round-robin over 8 XCDs)
    const int per = gridDim.x / 8;
    bid = (bid % 8) * per + bid / 8;
  }
  const int m0 = (bid / tiles_n) * BM;
  const int n0 = (bid % tiles_n) * BN;
  const int lane = threadIdx.x % cm::kWave;
  const int wave = threadIdx.x / cm::kWave;
  const int wm = wave / WN, wn = wave % WN;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  TileLoad<BM> la;
  TileLoad<BN> lb;
  la.load(A, lda, m0, M, 0, K);
  lb.load(B, ldb, n0, N, 0, K);
  la.store(lds[0]);
  lb.store(lds[0] + BM * kRowChunks);
  __syncthreads();

  const int kt_count = (K + kBK - 1) / kBK;
  for (int kt = 0; kt < kt_count; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < kt_count;
    if (more) {
      la.load(A, lda, m0, M, (kt + 1) * kBK, K);
      lb.load(B, ldb, n0, N, (kt + 1) * kBK, K);
    }
    const uint4* As = lds[cur];
    const uint4* Bs = lds[cur] + BM * kRowChunks;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int ch = ks * 2 + lane / 32;
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = frag(As, wm * WTM + i * 32 + lane % 32, ch);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = frag(Bs, wn * WTN + j * 32 + lane % 32, ch);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(lds[cur ^ 1]);
      lb.store(lds[cur ^ 1] + BM * kRowChunks);
    }
    __syncthreads();
  }
  epi.template apply<TM, TN>(acc, m0 + wm * WTM, n0 + wn * WTN, lane);
}

// Partial statistics of one (token, 128-column group): max, sum, dot, first argmax.
struct Partial {
  float max, sum, dot;
  int32_t best;
};

// ---------------------------------------------------------------------------------------------
// K1 epilogue: the tile is Z^T (rows = vocabulary columns of the chunk, cols = tokens).
struct EpiLogits {
  _Float16* s16;    // [n_tok, ld_s] fp16 logits of the chunk
  int64_t ld_s;
  int n_tok;
  int n_voc;        // valid columns of the chunk
  int64_t c0;       // first vocabulary index of the chunk
  Partial* part;    // [n_tok, n_groups]
  int n_groups;

  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb,
                                        int lane) const {
    static_assert(TM * 32 == kGroup, "a wavefront covers one 128-column group");
    const int half_id = lane / 32;
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int tok = nb + nt * 32 + lane % 32;
      cm::SoftmaxState st = cm::SoftmaxState::empty();
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int v0 = mb + mt * 32 + q * 8 + half_id * 4;
          union {
            uint2 u;
            _Float16 h[4];
          } pk;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            pk.h[j] = cm::from_f32<_Float16>(acc[mt][nt][q * 4 + j]);
            if (v0 + j < n_voc) st.push(static_cast<float>(pk.h[j]), c0 + v0 + j);
          }
          if (tok < n_tok) *reinterpret_cast<uint2*>(s16 + tok * ld_s + v0) = pk.u;
        }
      }
      st.merge(cm::shfl_xor_state(st, 32));
      if (half_id == 0 && tok < n_tok) {
        Partial p;
        p.max = st.max;
        p.sum = st.sum;
        p.dot = st.dot;
        p.best = static_cast<int32_t>(st.best == 0x7fffffffffffffffLL ? -1 : st.best);
        part[static_cast<int64_t>(tok) * n_groups + mb / kGroup] = p;
      }
    }
  }
};

// K3 epilogue: the tile is G (rows = tokens, cols = hidden units).
struct EpiGrad {
  float* grad;         // [n_tok, hidden] fp32, row stride ld_g
  int64_t ld_g;
  int n_tok;
  int hidden;
  const float* factor;  // [n_tok]
  int first;            // first chunk: G = acc

  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb,
                                        int lane) const {
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tok = mb + mt * 32 + (r / 4) * 8 + (lane / 32) * 4 + (r % 4);
        if (tok >= n_tok) continue;
        const float f = first ? 0.0f : factor[tok];
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          const int h = nb + nt * 32 + lane % 32;
          if (h >= hidden) continue;
          float* g = grad + static_cast<int64_t>(tok) * ld_g + h;
          *g = first ? acc[mt][nt][r] : *g * f + acc[mt][nt][r];
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------------------------
// Row state across chunks (structure of arrays, n_tok each).
struct RowState {
  float* max;
  float* sum;
  float* dot;
  int32_t* best;
  float* label_logit;
  float* lse;     // running log-sum-exp after the last merged chunk
  float* factor;  // e^{lse_before - lse_after} of the last merged chunk
};

// K2: merge the chunk's partials; record label logit and factor; optionally P in place.
__global__ __launch_bounds__(kStatThreads) void lmh_rows_kernel(
    _Float16* __restrict__ s16, int64_t ld_s, const Partial* __restrict__ part, int n_groups,
    RowState rs, const int64_t* __restrict__ target, int n_voc, int64_t c0, int first,
    int write_p) {
  const int row = blockIdx.x;
  cm::SoftmaxState st = cm::SoftmaxState::empty();
  const int n_valid = (n_voc + kGroup - 1) / kGroup;  // groups K1 wrote for this chunk
  for (int g = threadIdx.x; g < n_valid; g += kStatThreads) {
    const Partial p = part[static_cast<int64_t>(row) * n_groups + g];
    if (p.best >= 0) {
      cm::SoftmaxState q{p.max, p.sum, p.dot, static_cast<int64_t>(p.best)};
      st.merge(q);
    }
  }
  __shared__ cm::SoftmaxState s_part[kStatThreads / cm::kWave];
  st = cm::block_merge<kStatThreads>(st, s_part);
  cm::SoftmaxState prev = cm::SoftmaxState::empty();
  if (!first) {
    prev.max = rs.max[row];
    prev.sum = rs.sum[row];
    prev.dot = rs.dot[row];
    prev.best = rs.best[row];
  }
  const float lse_prev = first ? -__builtin_huge_valf() : prev.lse();
  cm::SoftmaxState now = prev;
  now.merge(st);
  const float lse_now = now.lse();
  const int64_t t = target[row];
  const bool labelled = t != -100;
  const int64_t local = t - c0;
  const bool hit = labelled && local >= 0 && local < n_voc;
  _Float16* zrow = s16 + static_cast<int64_t>(row) * ld_s;
  if (threadIdx.x == 0) {
    rs.max[row] = now.max;
    rs.sum[row] = now.sum;
    rs.dot[row] = now.dot;
    rs.best[row] = static_cast<int32_t>(now.best);
    rs.lse[row] = lse_now;
    rs.factor[row] = first ? 0.0f : cm::exp_f(lse_prev - lse_now);
    if (hit) rs.label_logit[row] = static_cast<float>(zrow[local]);
  }
  if (!write_p) return;
  __syncthreads();  // the label logit is read before the row is overwritten
  const int n8 = n_voc / 8;
  for (int i = threadIdx.x; i < n8; i += kStatThreads) {
    union {
      uint4 u;
      _Float16 h[8];
    } v;
    v.u = *reinterpret_cast<const uint4*>(zrow + 8 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = labelled ? cm::exp_f(static_cast<float>(v.h[e]) - lse_now) * kPScale : 0.0f;
      v.h[e] = cm::from_f32<_Float16>(p);
    }
    *reinterpret_cast<uint4*>(zrow + 8 * i) = v.u;
  }
  for (int c = n8 * 8 + threadIdx.x; c < n_voc; c += kStatThreads) {
    const float p = labelled ? cm::exp_f(static_cast<float>(zrow[c]) - lse_now) * kPScale : 0.0f;
    zrow[c] = cm::from_f32<_Float16>(p);
  }
}

// K4: final per-row outputs; gradient G = scale * (G / 1024 - W[t]) for labelled rows, else 0.
__global__ __launch_bounds__(kStatThreads) void lmh_final_kernel(
    RowState rs, const int64_t* __restrict__ target, int64_t vocab, float* __restrict__ loss,
    float* __restrict__ entropy, int32_t* __restrict__ correct, float* __restrict__ grad,
    int64_t ld_g, const _Float16* __restrict__ weight, int64_t ld_w, int hidden,
    float grad_scale) {
  const int row = blockIdx.x;
  const int64_t t = target[row];
  const bool labelled = t != -100;
  const bool in_range = t >= 0 && t < vocab;
  if (threadIdx.x == 0) {
    cm::SoftmaxState st{rs.max[row], rs.sum[row], rs.dot[row], rs.best[row]};
    const float lse = st.lse();
    const float zt = in_range ? rs.label_logit[row] : __builtin_nanf("");
    loss[row] = labelled ? lse - zt : 0.0f;
    entropy[row] = lse - st.dot / st.sum;
    correct[row] = labelled && st.best == t ? 1 : 0;
  }
  if (grad == nullptr) return;
  float* g = grad + static_cast<int64_t>(row) * ld_g;
  const _Float16* w = weight + (in_range ? t : 0) * ld_w;
  for (int h = threadIdx.x; h < hidden; h += kStatThreads) {
    g[h] = labelled && in_range
               ? grad_scale * (g[h] * (1.0f / kPScale) - static_cast<float>(w[h]))
               : (labelled ? __builtin_nanf("") : 0.0f);
  }
}

// W^T chunk: out[h, v] = W[c0 + v, h] for v < n_voc (64 x 64 tiles through LDS).
__global__ __launch_bounds__(kStatThreads) void lmh_transpose_kernel(
    const _Float16* __restrict__ w, int64_t ld_w, int64_t c0, int n_voc, int hidden,
    _Float16* __restrict__ wt, int64_t ld_t) {
  __shared__ _Float16 tile[64][66];
  const int v0 = blockIdx.x * 64, h0 = blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += kStatThreads) {
    const int r = i / 64, c = i % 64;
    const int v = v0 + r, h = h0 + c;
    tile[r][c] = (v < n_voc && h < hidden) ? w[(c0 + v) * ld_w + h] : _Float16(0);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += kStatThreads) {
    const int r = i / 64, c = i % 64;  // r: hidden, c: vocabulary
    const int h = h0 + r, v = v0 + c;
    if (h < hidden && v < ld_t) wt[static_cast<int64_t>(h) * ld_t + v] = tile[c][r];
  }
}

// ---------------------------------------------------------------------------------------------
// Workspace layout.
constexpr int kBM1 = 256, kBN1 = 256;  // K1 tiles (vocabulary x tokens)
constexpr int kBM3 = 128, kBN3 = 128;  // K3 tiles (tokens x hidden)

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

int64_t default_chunk(int64_t n_rows, int64_t vocab) {
  // Keep the fp16 chunk at <= 64 MiB so chunk, weight chunk and its transpose fit in the
  // 256 MB Infinity Cache; at least 4096 columns.
  int64_t c = (int64_t{32} << 20) / (n_rows > 0 ? n_rows : 1);
  c = c / kBM1 * kBM1;
  if (c < 4096) c = 4096;
  if (c > 65536) c = 65536;
  return c < vocab ? c : round_up(vocab, kBM1);
}

struct Layout {
  int64_t chunk, ld_s, n_groups, ld_t;
  int64_t off_s16, off_part, off_rows, off_wt, total;
};

Layout layout(int64_t n_rows, int64_t vocab, int hidden, int64_t chunk, bool need_wt) {
  Layout L;
  L.chunk = chunk > 0 ? round_up(chunk, kBM1) : default_chunk(n_rows, vocab);
  if (L.chunk > round_up(vocab, kBM1)) L.chunk = round_up(vocab, kBM1);
  L.ld_s = L.chunk;
  L.n_groups = L.ld_s / kGroup;
  L.ld_t = L.chunk;
  int64_t off = 0;
  L.off_s16 = off;
  off += round_up(n_rows * L.ld_s * 2, 256);
  L.off_part = off;
  off += round_up(n_rows * L.n_groups * static_cast<int64_t>(sizeof(Partial)), 256);
  L.off_rows = off;
  off += 8 * round_up(n_rows * 4, 256);
  L.off_wt = off;
  if (need_wt) off += round_up(static_cast<int64_t>(hidden) * L.ld_t * 2, 256);
  L.total = off;
  return L;
}

}  // namespace

extern "C" int64_t cm_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab, int hidden_size,
                                                int64_t chunk_cols) {
  if (n_rows <= 0 || vocab <= 0 || hidden_size <= 0) return 0;
  return layout(n_rows, vocab, hidden_size, chunk_cols, true).total;
}

extern "C" int cm_lmhead_ce(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
                            const void* weight_t, int64_t ld_wt, const int64_t* target,
                            int64_t n_rows, int64_t vocab, int hidden_size, int64_t chunk_cols,
                            float* loss, float* entropy, int32_t* correct, float* grad,
                            float grad_scale, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  CM_CHECK_ARG(n_rows >= 0 && vocab > 0 && hidden_size > 0 && chunk_cols >= 0);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(hidden && weight && target && loss && entropy && correct && workspace);
  CM_CHECK_ARG(n_rows < (int64_t{1} << 31) && vocab < (int64_t{1} << 31));
  // 16-byte tile rows: hidden size, leading dimensions and bases multiples of 8 fp16.
  CM_CHECK_ARG(hidden_size % 8 == 0 && ld_h % 8 == 0 && ld_w % 8 == 0 && ld_h >= hidden_size &&
               ld_w >= hidden_size && cm::aligned(hidden, 16) && cm::aligned(weight, 16));
  if (weight_t) CM_CHECK_ARG(ld_wt >= vocab && ld_wt % 8 == 0 && cm::aligned(weight_t, 16));
  const bool want_grad = grad != nullptr;
  const Layout L = layout(n_rows, vocab, hidden_size, chunk_cols, want_grad && !weight_t);
  CM_CHECK_ARG(workspace_bytes >= L.total && cm::aligned(workspace, 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  _Float16* s16 = reinterpret_cast<_Float16*>(ws + L.off_s16);
  Partial* part = reinterpret_cast<Partial*>(ws + L.off_part);
  const int64_t rstride = round_up(n_rows * 4, 256);
  char* rb = ws + L.off_rows;
  RowState rs{reinterpret_cast<float*>(rb), reinterpret_cast<float*>(rb + rstride),
              reinterpret_cast<float*>(rb + 2 * rstride), reinterpret_cast<int32_t*>(rb + 3 * rstride),
              reinterpret_cast<float*>(rb + 4 * rstride), reinterpret_cast<float*>(rb + 5 * rstride),
              reinterpret_cast<float*>(rb + 6 * rstride)};
  _Float16* wt_ws = reinterpret_cast<_Float16*>(ws + L.off_wt);
  const _Float16* H16 = static_cast<const _Float16*>(hidden);
  const _Float16* W16 = static_cast<const _Float16*>(weight);
  const int n_tok = static_cast<int>(n_rows);

  for (int64_t c0 = 0; c0 < vocab; c0 += L.chunk) {
    const int n_voc = static_cast<int>(vocab - c0 < L.chunk ? vocab - c0 : L.chunk);
    const bool first = c0 == 0;
    // K1: Z^T tile = W_c H^T
    {
      const int tiles_m = (n_voc + kBM1 - 1) / kBM1;
      const int tiles_n = (n_tok + kBN1 - 1) / kBN1;
      const int grid = tiles_m * tiles_n;
      EpiLogits epi{s16, L.ld_s, n_tok, n_voc, c0, part, static_cast<int>(L.n_groups)};
      hipLaunchKernelGGL((gemm_nt<kBM1, kBN1, 2, 2, EpiLogits>), dim3(grid), dim3(kThreads), 0, s,
                         W16 + c0 * ld_w, ld_w, n_voc, H16, ld_h, n_tok, hidden_size,
                         grid % 8 == 0 ? 1 : 0, epi);
      int st = cm::launch_status();
      if (st) return st;
    }
    // K2: running statistics (+ P in place)
    hipLaunchKernelGGL(lmh_rows_kernel, dim3(n_tok), dim3(kStatThreads), 0, s, s16, L.ld_s,
                       part, static_cast<int>(L.n_groups), rs, target, n_voc, c0, first ? 1 : 0,
                       want_grad ? 1 : 0);
    int st = cm::launch_status();
    if (st) return st;
    if (!want_grad) continue;
    // K3: G = G * factor + P W_c, with B = W_c^T rows (hidden) x vocabulary
    const _Float16* wt;
    int64_t ldt;
    if (weight_t) {
      wt = static_cast<const _Float16*>(weight_t) + c0;
      ldt = ld_wt;
    } else {
      dim3 tgrid((n_voc + 63) / 64, (hidden_size + 63) / 64);
      hipLaunchKernelGGL(lmh_transpose_kernel, tgrid, dim3(kStatThreads), 0, s, W16, ld_w, c0,
                         n_voc, hidden_size, wt_ws, L.ld_t);
      st = cm::launch_status();
      if (st) return st;
      wt = wt_ws;
      ldt = L.ld_t;
    }
    {
      const int tiles_m = (n_tok + kBM3 - 1) / kBM3;
      const int tiles_n = (hidden_size + kBN3 - 1) / kBN3;
      const int grid = tiles_m * tiles_n;
      EpiGrad epi{grad, hidden_size, n_tok, hidden_size, rs.factor, first ? 1 : 0};
      hipLaunchKernelGGL((gemm_nt<kBM3, kBN3, 2, 2, EpiGrad>), dim3(grid), dim3(kThreads), 0, s,
                         s16, L.ld_s, n_tok, wt, ldt, hidden_size, n_voc, grid % 8 == 0 ? 1 : 0,
                         epi);
      st = cm::launch_status();
      if (st) return st;
    }
  }
  hipLaunchKernelGGL(lmh_final_kernel, dim3(n_tok), dim3(kStatThreads), 0, s, rs, target, vocab,
                     loss, entropy, correct, grad, static_cast<int64_t>(hidden_size), W16, ld_w,
                     hidden_size, grad_scale);
  return cm::launch_status();
}
