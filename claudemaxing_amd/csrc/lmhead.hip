// Fused LM head + cross-entropy with per-row loss, entropy, accuracy and the hidden-state
// gradient (gfx950, fp16 MFMA with fp32 accumulation).
//
// Reproduces _FusedHeadLoss of the reference (solution/lm_head_loss.py:192-254: per vocabulary
// chunk torch.mm -> lm_head_vocab_chunk_kernel (108-160) -> torch.mm, then the label fix-up
// 230-236). The vocabulary is walked in chunks of C columns; per chunk, on the caller's stream:
//
//   K1 logits   Z^T = W_c H^T on the matrix cores (csrc/gemm_lds.h). The epilogue rounds every
//               logit to fp16 (the base path's fp16 logits) and reduces each token's logits of
//               the wavefront's 128-column vocabulary group to partial online-softmax statistics
//               (group max m_g, sum e^{z-m_g}, sum e^{z-m_g} z, first argmax) straight from the
//               accumulators: in the transposed tile a lane holds the logits of one token. It
//               stores E = fp16(e^{z - m_g}) for the gradient, and the label's logit.
//   K2 rows     per token: merge the partials into the running statistics, record the running
//               log-sum-exp and the rescale factor e^{lse_before - lse_after}, and turn each
//               group max into the group's probability scale s_g = e^{m_g - lse} * 1024 (zero
//               for unlabelled tokens).
//   K3 grad     G_s = G_s * factor + P W_c for K-slices s of the chunk (split-K over separate fp32
//               accumulators so the grid fills the chip), on the matrix cores, where
//               P = E * s_g (= e^{z - lse} * 1024 in fp16) is formed from each A fragment with
//               packed fp16 multiplies between the LDS read and the MFMA. The power-of-two scale
//               keeps the small probabilities of a 152K vocabulary out of fp16's subnormal
//               range.
//   K4 final    (after the last chunk) lse, loss, entropy, correct; G = scale (sum_s G_s / 1024
//               + (p_t - 1) W_t): K2 zeroes the label's entry of E, so the label's coefficient
//               is applied only here, in fp32.
//
// The full [tokens, vocab] logits never exist: one fp16 chunk of E (at most 1 GiB) lives in the
// workspace. The chunk and the transposed weight are stored in 64-column panels
// ([C/64][tokens][64], [V/64][H][64]) so that every K3 operand tile is one contiguous 16 KiB
// read.
#include <mutex>

#include "common.h"
#include "gemm_lds.h"
#include "softmax_state.h"

namespace {

using cm::gemm::Blocked64;
using cm::gemm::floatx16;
using cm::gemm::half8;
using cm::gemm::RowMajor;

constexpr int kPanel = 64;          // columns per panel of the blocked layouts
// Logit given to vocabulary rows past a chunk's last column in K1's epilogue: below every fp16
// value (and finite, so that e^{z - m} z is 0, not NaN).
constexpr float kNoLogit = -3.0e38f;
constexpr float kPScale = 1024.0f;  // P16 = fp16(p * kPScale)
constexpr int kStatThreads = 256;
constexpr int kMaxSplit = 8;

// Tile configurations: BM, BN, wavefront grid WM x WN, stage depth BK, LDS ring stages, and the
// minimum wavefronts per SIMD for __launch_bounds__ (which caps the registers per wavefront:
// 2 gives 256, 1 gives 512). Variant 0 is the default; variant 1 of each is the alternative
// measured beside it (a deeper ring of 32-column stages; for K3 four wavefronts of 128 x 96).
#ifndef CM_LMH_K1
#define CM_LMH_K1 0
#endif
#ifndef CM_LMH_K3
#define CM_LMH_K3 0
#endif
#if CM_LMH_K1 == 1
constexpr int kBM1 = 256, kBN1 = 256, kWM1 = 2, kWN1 = 4, kBK1 = 32, kST1 = 4, kOcc1 = 2;
#else
constexpr int kBM1 = 256, kBN1 = 256, kWM1 = 2, kWN1 = 4, kBK1 = 64, kST1 = 2, kOcc1 = 2;
#endif
#if CM_LMH_K3 == 1
constexpr int kBM3 = 256, kBN3 = 192, kWM3 = 2, kWN3 = 2, kBK3 = 32, kST3 = 4, kOcc3 = 1;
#elif CM_LMH_K3 == 2
constexpr int kBM3 = 256, kBN3 = 256, kWM3 = 2, kWN3 = 4, kBK3 = 64, kST3 = 2, kOcc3 = 2;
#else
constexpr int kBM3 = 256, kBN3 = 192, kWM3 = 4, kWN3 = 2, kBK3 = 64, kST3 = 2, kOcc3 = 2;
#endif
constexpr int kThreads1 = kWM1 * kWN1 * cm::kWave;
constexpr int kThreads3 = kWM3 * kWN3 * cm::kWave;
constexpr int kGroup = kBM1 / kWM1;  // vocabulary columns per partial-statistics group
constexpr int kEpiRows = kGroup / 2;  // group rows one lane of K1's epilogue holds per token
static_assert(kGroup % kPanel == 0, "a statistics group is whole panels");

__device__ __forceinline__ int64_t panel_index(int64_t row, int64_t col, int64_t rows) {
  return ((col / kPanel) * rows + row) * kPanel + col % kPanel;
}

// Partial statistics of one (token, group): group max, sum e^{z - max}, sum e^{z - max} z, first
// argmax as a vocabulary index (-1 when the group holds no valid column).
struct Partial {
  float max, sum, dot;
  int32_t best;
};

// ---------------------------------------------------------------------------------------------
// K1 epilogue: the tile is Z^T (rows = vocabulary columns of the chunk, cols = tokens). A
// wavefront's rows are one statistics group of kGroup columns. E is staged in the LDS in the
// output's panel layout and written with 16-byte stores, 1 KiB contiguous per wavefront
// instruction: the tile's BM vocabulary rows are BM / 64 panels, and in each the BN tokens are one
// contiguous span of BN x 128 bytes.
struct EpiProbs {
  static constexpr int kTN = kBN1 / kWN1 / 32;
  _Float16* e16;        // chunk of E = fp16(e^{z - m_g}), panels [C/64][n_tok][64]
  int n_tok;
  int n_voc;            // valid columns of the chunk
  int64_t c0;           // first vocabulary index of the chunk
  Partial* part;        // [n_tok, n_groups]
  int n_groups;
  const int64_t* target;
  _Float16* label_z;    // [n_tok][2][64]: the label group's fp16 logits, lane by lane
  int store;            // write E (the gradient needs it)
  int64_t tgt[kTN];     // targets of the lane's tokens, loaded before the main loop

  // 16-byte chunk slot of (token t, chunk c) within the staging rows of panel p: rows of 128
  // bytes, chunk XOR-swizzled by the token so that 16 consecutive tokens hit distinct banks.
  static __device__ __forceinline__ int stage_slot(int p, int t, int c) {
    return (p * kBN1 + t) * 8 + (c ^ ((t >> 1) & 7));
  }

  template <int TM, int TN>
  __device__ __forceinline__ void prepare(int, int nb, int lane) {
    static_assert(TN == kTN, "epilogue configured for K1's wavefront tile");
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int tok = nb + nt * 32 + lane % 32;
      tgt[nt] = tok < n_tok ? target[tok] : int64_t{-100};
    }
  }

  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb, int lane,
                                        uint4* lds) {
    static_assert(TM * 32 == kGroup, "a wavefront covers one statistics group");
    static_assert(kBM1 * kBN1 * 2 <= kST1 * (kBM1 + kBN1) * kBK1 * 2,
                  "the E tile is staged in the LDS ring");
    const int half_id = lane / 32;
    const int m0 = mb - mb % kBM1, n0 = nb - nb % kBN1;  // tile origin
    // accumulator element e of a lane is vocabulary row mb + vrow(e)
    auto vrow = [&](int e) { return (e / 16) * 32 + ((e % 16) / 4) * 8 + half_id * 4 + e % 4; };
    if (store) cm::gemm::lds_barrier();  // every wavefront is done reading the last stage
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int tok = nb + nt * 32 + lane % 32;
      const bool tok_ok = tok < n_tok;
      // fp16 logits of this lane's token, in place of its accumulators (a separate array of 64
      // values made the epilogue spill); rows past the chunk's last column get kNoLogit, which
      // no fp16 logit reaches and whose e^{z - m} is 0, so the loops below need no validity
      // test per element
#define Z(e) acc[(e) / 16][nt][(e) % 16]
#pragma unroll
      for (int e = 0; e < TM * 16; ++e)
        Z(e) = mb + vrow(e) < n_voc ? static_cast<float>(cm::from_f32<_Float16>(Z(e))) : kNoLogit;
      // group max and first argmax over both halves of the wavefront (branch-free)
      float m = kNoLogit;
      int best = -1;
#pragma unroll
      for (int e = 0; e < TM * 16; ++e) {
        const bool take = Z(e) > m;
        m = take ? Z(e) : m;
        best = take ? mb + vrow(e) : best;
      }
      const float m_o = __shfl_xor(m, 32, cm::kWave);
      const int best_o = __shfl_xor(best, 32, cm::kWave);
      const bool other = m_o > m || (m_o == m && best_o >= 0 && (best < 0 || best_o < best));
      best = other ? best_o : best;
      // a group with no usable logit: every e^{z - mg} below is then 0
      const float mg = best < 0 ? __builtin_huge_valf() : (other ? m_o : m);
      // The token's label falls in this group (rare): both lanes of the token copy their 64
      // fp16 logits out, and K2 takes the label's logit and the group's sum over its other
      // columns from them (that sum, kept apart from the label's term, is exact where the
      // label dominates its group; forming it here raised the live set past the register file).
      const int64_t local = tgt[nt] - c0 - mb;
      if (tok_ok && local >= 0 && local < kGroup && mb + local < n_voc) {
        _Float16* dst = label_z + (static_cast<int64_t>(tok) * 2 + half_id) * (TM * 16);
#pragma unroll
        for (int e = 0; e < TM * 16; e += 4) {
          union {
            uint2 u;
            _Float16 h[4];
          } pk;
#pragma unroll
          for (int j = 0; j < 4; ++j) pk.h[j] = static_cast<_Float16>(Z(e + j));  // exact
          *reinterpret_cast<uint2*>(dst + e) = pk.u;
        }
      }
      // E = e^{z - m_g} (in place of z) and the sums, relative to the group max
      float s = 0.0f, d = 0.0f;
#pragma unroll
      for (int e = 0; e < TM * 16; ++e) {
        const float x = cm::exp_f(Z(e) - mg);  // 0 for kNoLogit rows, so x z = -0 there
        s += x;
        d += x * Z(e);
        Z(e) = x;
      }
      s += __shfl_xor(s, 32, cm::kWave);
      d += __shfl_xor(d, 32, cm::kWave);
      if (store) {
        // stage: 4 consecutive vocabulary rows (8 bytes) per (mt, q)
        const int t = tok - n0;
#pragma unroll
        for (int mt = 0; mt < TM; ++mt) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            union {
              uint2 u;
              _Float16 h[4];
            } pk;
#pragma unroll
            for (int j = 0; j < 4; ++j) pk.h[j] = cm::from_f32<_Float16>(Z(mt * 16 + q * 4 + j));
            const int v = mb - m0 + mt * 32 + q * 8 + half_id * 4;  // tile-local vocabulary row
            uint2* dst = reinterpret_cast<uint2*>(lds + stage_slot(v / 64, t, (v % 64) / 8));
            dst[half_id] = pk.u;
          }
        }
      }
#undef Z
      if (half_id == 0 && tok_ok) {
        Partial p;
        p.max = best < 0 ? -__builtin_huge_valf() : mg;
        p.sum = s;
        p.dot = d;
        p.best = best >= 0 ? static_cast<int32_t>(c0 + best) : -1;
        part[static_cast<int64_t>(tok) * n_groups + mb / kGroup] = p;
      }
    }
    if (!store) return;
    cm::gemm::lds_barrier();
    // copy out: slot = (p * BN + t) * 8 + physical chunk; 8 consecutive threads = one token row
    constexpr int kSlots = kBM1 / 64 * kBN1 * 8;
    for (int slot = threadIdx.x; slot < kSlots; slot += kThreads1) {
      const int row = slot / 8, pc = slot % 8;
      const int p = row / kBN1, t = row % kBN1;
      if (n0 + t >= n_tok) continue;
      const int c = pc ^ ((t >> 1) & 7);
      const int64_t dst = ((static_cast<int64_t>((m0 / 64) + p) * n_tok + n0 + t) * 64) + c * 8;
      *reinterpret_cast<uint4*>(e16 + dst) = lds[slot];
    }
  }
};

// K3 epilogue: the tile is G (rows = tokens, cols = hidden units).
struct EpiGrad {
  float* grad;          // [n_tok, hidden] fp32 accumulator of this K-slice
  int n_tok;
  int hidden;
  const float* factor;  // [n_tok]
  int first;            // first chunk: G = acc

  template <int TM, int TN>
  __device__ __forceinline__ void prepare(int, int, int) {}

  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb, int lane,
                                        uint4*) const {
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
          float* g = grad + static_cast<int64_t>(tok) * hidden + h;
          *g = first ? acc[mt][nt][r] : *g * f + acc[mt][nt][r];
        }
      }
    }
  }
};

// __launch_bounds__'s second argument is the minimum number of wavefronts per SIMD, which caps
// the registers per wavefront accordingly.
template <class Epi, int BM, int BN, int WM, int WN, int BK, int ST, int OCC>
__global__ __launch_bounds__(WM * WN * cm::kWave, OCC) void lmh_gemm1(RowMajor A, RowMajor B,
                                                                       int remap, Epi epi) {
  __shared__ uint4 lds[ST * (BM + BN) * (BK / 8)];
  int tm, tn;
  cm::gemm::tile_of_block((B.rows + BN - 1) / BN, remap, tm, tn);
  cm::gemm::gemm_lds<BM, BN, WM, WN, BK, ST>(A, B, 0, A.k_len, tm, tn, epi, lds);
}

// K3's A-fragment transform: E (fp16 e^{z - m_g}) times the (token, group) scale
// s_g = e^{m_g - lse} * 1024 (0 for unlabelled tokens) gives P16 = e^{z - lse} * 1024. The
// scales of the next stage are loaded one stage ahead; each A fragment (8 columns of one token,
// all inside one group) then costs four packed fp16 multiplies.
template <int TM>
struct ScaleP {
  const float* scale;  // [groups][n_tok]
  int n_tok;
  int row = 0;
  float nxt[TM];
  _Float16 cur[TM];

  __device__ __forceinline__ void bind(int r) { row = r; }
  __device__ __forceinline__ void prefetch(int k0) {
    const float* s = scale + static_cast<int64_t>(k0 / kGroup) * n_tok;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = row + 32 * i;
      nxt[i] = r < n_tok ? s[r] : 0.0f;
    }
  }
  __device__ __forceinline__ void advance() {
#pragma unroll
    for (int i = 0; i < TM; ++i) cur[i] = static_cast<_Float16>(nxt[i]);
  }
  __device__ __forceinline__ half8 apply(half8 f, int i) const { return f * cur[i]; }
};

// K3: blockIdx.y is the K-slice; each slice accumulates into its own buffer.
struct GradSlices {
  float* g[kMaxSplit];
};

template <int BM, int BN, int WM, int WN, int BK, int ST, int OCC>
__global__ __launch_bounds__(WM * WN * cm::kWave, OCC) void lmh_gemm3(
    Blocked64 A, Blocked64 B, int k_slice, int remap, GradSlices out, int n_tok, int hidden,
    const float* factor, int first, const float* scale) {
  __shared__ uint4 lds[ST * (BM + BN) * (BK / 8)];
  int tm, tn, s;
  cm::gemm::tile_of_block_2d((B.rows + BN - 1) / BN, remap, tm, tn, s);
  const int k_begin = s * k_slice;
  // An empty slice still runs the epilogue (with zero accumulators) so that its buffer is
  // initialised on the first chunk and rescaled on later ones.
  const int k_end = max(k_begin, min(A.k_len, k_begin + k_slice));
  EpiGrad epi{out.g[s], n_tok, hidden, factor, first};
  ScaleP<BM / WM / 32> xp{scale, n_tok, 0, {}, {}};  // nxt / cur are filled by prefetch
  cm::gemm::gemm_lds<BM, BN, WM, WN, BK, ST>(A, B, k_begin, k_end, tm, tn, epi, lds, xp);
}

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
  float* off;  // running sum of e^{z - max} over the columns other than the label
};
constexpr int kRowArrays = 8;  // row-state arrays in the workspace, one per field
static_assert(sizeof(RowState) == kRowArrays * sizeof(void*),
              "RowState holds exactly one workspace array per field");

// The row state's arrays, laid out one after another from `base`, `stride` bytes apart. Every
// field is assigned by name here; `complete` says none was left null.
RowState row_state(char* base, int64_t stride) {
  auto at = [&](int i) { return reinterpret_cast<float*>(base + i * stride); };
  RowState r;
  r.max = at(0);
  r.sum = at(1);
  r.dot = at(2);
  r.best = reinterpret_cast<int32_t*>(at(3));
  r.label_logit = at(4);
  r.lse = at(5);
  r.factor = at(6);
  r.off = at(7);
  return r;
}

bool complete(const RowState& r) {
  const void* const* p = reinterpret_cast<const void* const*>(&r);
  for (int i = 0; i < kRowArrays; ++i)
    if (p[i] == nullptr) return false;
  return true;
}

// The running statistics with the off-label mass beside them: `off` is the sum of e^{z - max}
// over every column but the label, rescaled with the maximum like `sum`. The label's
// probability is then p_t = 1 - off / sum exactly, however close to 1 it is (1 - p_t computed
// from an fp32 log-sum-exp would be quantized to the 2^-24 steps of the sum near 1).
struct OffState {
  cm::SoftmaxState st;
  float off;

  static __device__ __forceinline__ OffState empty() {
    return OffState{cm::SoftmaxState::empty(), 0.0f};
  }
  __device__ __forceinline__ void merge(const OffState& o) {
    if (o.st.max == -__builtin_huge_valf()) return;
    if (st.max == -__builtin_huge_valf()) {
      *this = o;
      return;
    }
    const float m = fmaxf(st.max, o.st.max);
    off = off * cm::exp_f(st.max - m) + o.off * cm::exp_f(o.st.max - m);
    st.merge(o.st);
  }
};

// Merge the states of all lanes of a THREADS-lane workgroup; every lane gets the result.
template <int THREADS>
__device__ __forceinline__ OffState block_merge_off(OffState s, OffState* part) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) {
    OffState o{cm::shfl_xor_state(s.st, d), __shfl_xor(s.off, d, cm::kWave)};
    s.merge(o);
  }
  const int wave = threadIdx.x / cm::kWave;
  if (threadIdx.x % cm::kWave == 0) part[wave] = s;
  __syncthreads();
  OffState r = part[0];
#pragma unroll
  for (int i = 1; i < THREADS / cm::kWave; ++i) r.merge(part[i]);
  return r;
}

// K2: merge the chunk's partials into the running state; the factor; with a scale array, the
// group scales s_g = e^{m_g - lse} * 1024 of labelled tokens ([groups][n_tok], 0 otherwise),
// and the label's own entry of E set to 0 when the label falls in this chunk: the label's
// coefficient p_t - 1 is applied by K4 in fp32, so its near-1 probability never enters the
// fp32 accumulators (a ~1024 W_t term there would cancel against -1024 W_t only at the end,
// losing the small difference 1 - p_t of a confident label to the accumulators' rounding).
__global__ __launch_bounds__(kStatThreads) void lmh_rows_kernel(
    const Partial* __restrict__ part, int n_groups, RowState rs,
    const int64_t* __restrict__ target, int n_tok, int64_t c0, int n_voc, int first,
    float* __restrict__ scale, _Float16* __restrict__ e16, const _Float16* __restrict__ label_z) {
  const int row = blockIdx.x;
  const int64_t t = target[row];
  const bool labelled = t != -100;
  // the label's statistics group in this chunk, or -1
  const int64_t g_label = t >= c0 && t < c0 + n_voc ? (t - c0) / kGroup : -1;
  // From the label group's 128 fp16 logits (K1 copied them out lane by lane: entry e of the
  // lane in half h is group row (e/16)*32 + ((e%16)/4)*8 + 4h + e%4): the label's logit and the
  // group's sum of e^{z - m_g} over its other columns, relative to the group max as K1's sums
  // are. Rows past the chunk hold -inf.
  __shared__ float s_red[kStatThreads / cm::kWave];
  __shared__ float s_zt;
  float label_off = 0.0f;
  if (g_label >= 0) {  // uniform over the workgroup
    const int local = static_cast<int>(t - c0 - g_label * kGroup);
    const float mg = part[static_cast<int64_t>(row) * n_groups + g_label].max;
    float v = 0.0f;
    if (threadIdx.x < 2 * kEpiRows) {
      const int h = threadIdx.x / kEpiRows, e = threadIdx.x % kEpiRows;
      const int r = (e / 16) * 32 + ((e % 16) / 4) * 8 + h * 4 + e % 4;
      const float z = static_cast<float>(label_z[static_cast<int64_t>(row) * 2 * kEpiRows +
                                                 threadIdx.x]);
      if (r == local) s_zt = z;
      else v = cm::exp_f(z - mg);
    }
    v = cm::wave_sum(v);
    if (threadIdx.x % cm::kWave == 0) s_red[threadIdx.x / cm::kWave] = v;
    __syncthreads();
    for (int w = 0; w < kStatThreads / cm::kWave; ++w) label_off += s_red[w];
    if (threadIdx.x == 0) rs.label_logit[row] = s_zt;
  }
  OffState acc = OffState::empty();
  const int n_valid = (n_voc + kGroup - 1) / kGroup;  // groups K1 wrote for this chunk
  for (int g = threadIdx.x; g < n_valid; g += kStatThreads) {
    const Partial p = part[static_cast<int64_t>(row) * n_groups + g];
    if (p.best >= 0) {
      OffState q{{p.max, p.sum, p.dot, static_cast<int64_t>(p.best)},
                 g == g_label ? label_off : p.sum};
      acc.merge(q);
    }
  }
  __shared__ OffState s_part[kStatThreads / cm::kWave];
  acc = block_merge_off<kStatThreads>(acc, s_part);
  OffState now = OffState::empty();
  if (!first) {
    now.st = cm::SoftmaxState{rs.max[row], rs.sum[row], rs.dot[row], rs.best[row]};
    now.off = rs.off[row];
  }
  const float lse_prev = first ? -__builtin_huge_valf() : now.st.lse();
  now.merge(acc);
  const float lse_now = now.st.lse();
  if (threadIdx.x == 0) {
    rs.max[row] = now.st.max;
    rs.sum[row] = now.st.sum;
    rs.dot[row] = now.st.dot;
    rs.best[row] = static_cast<int32_t>(now.st.best);
    rs.off[row] = now.off;
    rs.lse[row] = lse_now;
    rs.factor[row] = first ? 0.0f : cm::exp_f(lse_prev - lse_now);
  }
  if (scale == nullptr) return;
  for (int g = threadIdx.x; g < n_valid; g += kStatThreads) {
    const float m = part[static_cast<int64_t>(row) * n_groups + g].max;
    scale[static_cast<int64_t>(g) * n_tok + row] =
        labelled ? cm::exp_f(m - lse_now) * kPScale : 0.0f;
  }
  if (threadIdx.x == 0 && g_label >= 0)
    e16[panel_index(row, t - c0, n_tok)] = static_cast<_Float16>(0.0f);
}

// K4: final per-row outputs; G = scale * (sum_s G_s / 1024 + (p_t - 1) W[t]) for labelled rows,
// else 0.
__global__ __launch_bounds__(kStatThreads) void lmh_final_kernel(
    RowState rs, const int64_t* __restrict__ target, int64_t vocab, float* __restrict__ loss,
    float* __restrict__ entropy, int32_t* __restrict__ correct, GradSlices gs, int n_split,
    const _Float16* __restrict__ weight, int64_t ld_w, int hidden, float grad_scale) {
  const int row = blockIdx.x;
  const int64_t t = target[row];
  const bool labelled = t != -100;
  const bool in_range = t >= 0 && t < vocab;
  if (threadIdx.x == 0) {
    cm::SoftmaxState st{rs.max[row], rs.sum[row], rs.dot[row], rs.best[row]};
    const float lse = st.lse();
    const float zt = in_range ? rs.label_logit[row] : __builtin_nanf("");
    // lse - z_t = ln(e^{z_t - M} + off) - (z_t - M) = log1p(off e^{M - z_t}): no cancellation
    // of two nearly equal logs when the label takes almost all of the probability. A label far
    // below the maximum (loss >= 30, where e^{M - z_t} could overflow) takes lse - z_t.
    const float gap = st.max - zt;
    loss[row] = !labelled ? 0.0f
                : gap < 30.0f ? cm::log1p_f(rs.off[row] * cm::exp_f(gap)) : lse - zt;
    entropy[row] = lse - st.dot / st.sum;
    correct[row] = labelled && st.best == t ? 1 : 0;
  }
  if (gs.g[0] == nullptr) return;
  const _Float16* w = weight + (in_range ? t : 0) * ld_w;
  const int64_t off = static_cast<int64_t>(row) * hidden;
  // The label's column was zeroed in E (K2), so the accumulators hold sum_{v != t} p_v W_v; the
  // label's whole coefficient p_t - 1 = -off / sum is applied here in fp32, with the relative
  // precision of the off-label mass however confident the label is.
  const float coef = labelled && in_range ? -rs.off[row] / rs.sum[row] : 0.0f;
  for (int h = threadIdx.x; h < hidden; h += kStatThreads) {
    float acc = gs.g[0][off + h];
    for (int s = 1; s < n_split; ++s) acc += gs.g[s][off + h];
    gs.g[0][off + h] = labelled && in_range
                           ? grad_scale * (acc * (1.0f / kPScale) + coef * static_cast<float>(w[h]))
                           : (labelled ? __builtin_nanf("") : 0.0f);
  }
}

// W_c^T in panels: out[p][h][j] = W[c0 + 64 p + j][h], zero for 64 p + j >= n_voc.
__global__ __launch_bounds__(kStatThreads) void lmh_transpose_kernel(
    const _Float16* __restrict__ w, int64_t ld_w, int64_t c0, int n_voc, int hidden,
    _Float16* __restrict__ wt) {
  __shared__ _Float16 tile[64][66];
  const int p = blockIdx.x, h0 = blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += kStatThreads) {
    const int r = i / 64, c = i % 64;  // r: vocabulary within the panel, c: hidden
    const int v = p * 64 + r, h = h0 + c;
    tile[r][c] = (v < n_voc && h < hidden) ? w[(c0 + v) * ld_w + h] : _Float16(0);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += kStatThreads) {
    const int r = i / 64, c = i % 64;  // r: hidden, c: vocabulary
    const int h = h0 + r;
    if (h < hidden) wt[(static_cast<int64_t>(p) * hidden + h) * 64 + c] = tile[c][r];
  }
}

// ---------------------------------------------------------------------------------------------
// Workspace layout.
int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

constexpr int64_t kChunkAlign = kBM1 > 256 ? kBM1 : 256;

int64_t default_chunk(int64_t n_rows, int64_t vocab) {
  // E chunk of at most 1 GiB (fp16, n_rows x C), whatever the vocabulary, split into equal
  // chunks. Fewer, larger chunks pay the per-chunk costs (launch ramps, each launch's partly
  // filled last wave of workgroups, the read-modify-write of the split-K gradient accumulators)
  // fewer times; measured at N = 2048, V = 151936: 38016 columns (4 chunks) 2.51 ms, 50688
  // (3) 2.51 ms, 75968 (2) 2.40 ms, one chunk 2.31 ms (a 622 MB E buffer, 0.2% of the HBM).
  const int64_t budget = (int64_t{512} << 20) / (n_rows > 0 ? n_rows : 1);  // columns
  int64_t c = budget / kChunkAlign * kChunkAlign;
  if (c < 4096) c = 4096;
  if (c >= vocab) return round_up(vocab, kChunkAlign);
  const int64_t n_chunks = (vocab + c - 1) / c;
  return round_up((vocab + n_chunks - 1) / n_chunks, kChunkAlign);
}

// K-slices of the gradient GEMM: as many as keep the grid within one workgroup per CU (256).
int n_split_for(int64_t n_rows, int hidden) {
  const int64_t tiles = ((n_rows + kBM3 - 1) / kBM3) * ((hidden + kBN3 - 1) / kBN3);
  int64_t s = 256 / (tiles > 0 ? tiles : 1);
  if (s < 1) s = 1;
  if (s > kMaxSplit) s = kMaxSplit;
  return static_cast<int>(s);
}

struct Layout {
  int64_t chunk, n_groups;
  int n_split;
  int64_t off_e16, off_part, off_rows, off_labz, off_scale, off_g, off_wt, total;
};

Layout layout(int64_t n_rows, int64_t vocab, int hidden, int64_t chunk, bool want_grad,
              bool need_wt) {
  Layout L;
  L.chunk = chunk > 0 ? round_up(chunk, kChunkAlign) : default_chunk(n_rows, vocab);
  if (L.chunk > round_up(vocab, kChunkAlign)) L.chunk = round_up(vocab, kChunkAlign);
  L.n_groups = L.chunk / kGroup;
  L.n_split = want_grad ? n_split_for(n_rows, hidden) : 1;
  int64_t off = 0;
  L.off_e16 = off;
  off += round_up(n_rows * L.chunk * 2, 256);
  L.off_part = off;
  off += round_up(n_rows * L.n_groups * static_cast<int64_t>(sizeof(Partial)), 256);
  L.off_rows = off;
  off += kRowArrays * round_up(n_rows * 4, 256);
  L.off_labz = off;
  off += round_up(n_rows * 2 * kEpiRows * 2, 256);
  L.off_scale = off;
  off += round_up(n_rows * L.n_groups * 4, 256);
  L.off_g = off;
  off += (L.n_split - 1) * round_up(n_rows * hidden * 4, 256);
  L.off_wt = off;
  if (need_wt) off += round_up(static_cast<int64_t>(hidden) * L.chunk * 2, 256);
  L.total = off;
  return L;
}

}  // namespace

extern "C" int64_t cm_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab, int hidden_size,
                                                int64_t chunk_cols) {
  if (n_rows <= 0 || vocab <= 0 || hidden_size <= 0) return 0;
  return layout(n_rows, vocab, hidden_size, chunk_cols, true, true).total;
}

namespace {

// Argument checks shared by both entry points (everything but the workspace).
bool args_ok(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
             const void* weight_t, const int64_t* target, int64_t n_rows, int64_t vocab,
             int hidden_size, int64_t chunk_cols, const float* loss, const float* entropy,
             const int32_t* correct) {
  if (!(n_rows > 0 && vocab > 0 && hidden_size > 0 && chunk_cols >= 0)) return false;
  if (!(hidden && weight && target && loss && entropy && correct)) return false;
  if (!(n_rows < (int64_t{1} << 31) && vocab < (int64_t{1} << 31))) return false;
  // 16-byte tile rows: hidden size, leading dimensions and bases multiples of 8 fp16.
  if (!(hidden_size % 8 == 0 && ld_h % 8 == 0 && ld_w % 8 == 0 && ld_h >= hidden_size &&
        ld_w >= hidden_size && cm::aligned(hidden, 16) && cm::aligned(weight, 16)))
    return false;
  return weight_t == nullptr || cm::aligned(weight_t, 16);
}

// The launches of one call (K1..K4 per chunk), on `ws` laid out as L; the arguments and the
// workspace's size and alignment have been checked.
int run_lmhead(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
               const void* weight_t, const int64_t* target, int64_t n_rows, int64_t vocab,
               int hidden_size, float* loss, float* entropy, int32_t* correct, float* grad,
               float grad_scale, char* ws, const Layout& L, hipStream_t s) {
  const bool want_grad = grad != nullptr;
  _Float16* e16 = reinterpret_cast<_Float16*>(ws + L.off_e16);
  Partial* part = reinterpret_cast<Partial*>(ws + L.off_part);
  float* scale = want_grad ? reinterpret_cast<float*>(ws + L.off_scale) : nullptr;
  const RowState rs = row_state(ws + L.off_rows, round_up(n_rows * 4, 256));
  if (!complete(rs)) return static_cast<int>(hipErrorInvalidValue);
  _Float16* label_z = reinterpret_cast<_Float16*>(ws + L.off_labz);
  GradSlices gs{};
  gs.g[0] = grad;
  for (int i = 1; i < L.n_split; ++i)
    gs.g[i] = reinterpret_cast<float*>(ws + L.off_g + (i - 1) * round_up(n_rows * hidden_size * 4, 256));
  _Float16* wt_ws = reinterpret_cast<_Float16*>(ws + L.off_wt);
  const _Float16* H16 = static_cast<const _Float16*>(hidden);
  const _Float16* W16 = static_cast<const _Float16*>(weight);
  const int n_tok = static_cast<int>(n_rows);

  for (int64_t c0 = 0; c0 < vocab; c0 += L.chunk) {
    const int n_voc = static_cast<int>(vocab - c0 < L.chunk ? vocab - c0 : L.chunk);
    const bool first = c0 == 0;
    // K1: Z^T tile = W_c H^T, statistics, E and the label logit
    {
      const int tiles_m = (n_voc + kBM1 - 1) / kBM1;
      const int tiles_n = (n_tok + kBN1 - 1) / kBN1;
      const int grid = tiles_m * tiles_n;
      RowMajor A{W16 + c0 * ld_w, ld_w, n_voc, hidden_size};
      RowMajor B{H16, ld_h, n_tok, hidden_size};
      EpiProbs epi{e16, n_tok, n_voc, c0, part, static_cast<int>(L.n_groups), target,
                   label_z, want_grad ? 1 : 0, {}};  // tgt: prepare()
      hipLaunchKernelGGL((lmh_gemm1<EpiProbs, kBM1, kBN1, kWM1, kWN1, kBK1, kST1, kOcc1>), dim3(grid),
                         dim3(kThreads1), 0, s, A, B, grid % 8 == 0 ? 1 : 0, epi);
      int st = cm::launch_status();
      if (st) return st;
    }
    // K2: running statistics and the group scales
    hipLaunchKernelGGL(lmh_rows_kernel, dim3(n_tok), dim3(kStatThreads), 0, s, part,
                       static_cast<int>(L.n_groups), rs, target, n_tok, c0, n_voc,
                       first ? 1 : 0, scale, e16, label_z);
    int st = cm::launch_status();
    if (st) return st;
    if (!want_grad) continue;
    // K3: G_s = G_s * factor + P W_c over K-slices, B = W_c^T in panels
    const _Float16* wt;
    if (weight_t) {
      wt = static_cast<const _Float16*>(weight_t) + (c0 / kPanel) * hidden_size * kPanel;
    } else {
      dim3 tgrid((n_voc + kPanel - 1) / kPanel, (hidden_size + 63) / 64);
      hipLaunchKernelGGL(lmh_transpose_kernel, tgrid, dim3(kStatThreads), 0, s, W16, ld_w, c0,
                         n_voc, hidden_size, wt_ws);
      st = cm::launch_status();
      if (st) return st;
      wt = wt_ws;
    }
    {
      const int tiles_m = (n_tok + kBM3 - 1) / kBM3;
      const int tiles_n = (hidden_size + kBN3 - 1) / kBN3;
      const int grid = tiles_m * tiles_n;
      const int panels = (n_voc + kPanel - 1) / kPanel;
      // slices are whole statistics groups, so a stage never straddles two group scales
      const int groups = (panels * kPanel + kGroup - 1) / kGroup;
      const int k_slice = ((groups + L.n_split - 1) / L.n_split) * kGroup;
      Blocked64 A{e16, n_tok, n_voc};
      Blocked64 B{wt, hidden_size, n_voc};
      hipLaunchKernelGGL((lmh_gemm3<kBM3, kBN3, kWM3, kWN3, kBK3, kST3, kOcc3>),
                         dim3(grid, L.n_split), dim3(kThreads3), 0, s, A, B, k_slice,
                         (grid * L.n_split) % 8 == 0 ? 1 : 0, gs, n_tok, hidden_size, rs.factor,
                         first ? 1 : 0,
                         scale);
      st = cm::launch_status();
      if (st) return st;
    }
  }
  GradSlices fin = want_grad ? gs : GradSlices{};
  hipLaunchKernelGGL(lmh_final_kernel, dim3(n_tok), dim3(kStatThreads), 0, s, rs, target, vocab,
                     loss, entropy, correct, fin, L.n_split, W16, ld_w, hidden_size, grad_scale);
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_lmhead_ce(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
                            const void* weight_t, const int64_t* target, int64_t n_rows,
                            int64_t vocab, int hidden_size, int64_t chunk_cols, float* loss,
                            float* entropy, int32_t* correct, float* grad, float grad_scale,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  CM_CHECK_ARG(n_rows >= 0);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(args_ok(hidden, ld_h, weight, ld_w, weight_t, target, n_rows, vocab, hidden_size,
                       chunk_cols, loss, entropy, correct));
  CM_CHECK_ARG(workspace != nullptr);
  const bool want_grad = grad != nullptr;
  const Layout L = layout(n_rows, vocab, hidden_size, chunk_cols, want_grad, want_grad && !weight_t);
  CM_CHECK_ARG(workspace_bytes >= L.total && cm::aligned(workspace, 256));
  return run_lmhead(hidden, ld_h, weight, ld_w, weight_t, target, n_rows, vocab, hidden_size,
                    loss, entropy, correct, grad, grad_scale, static_cast<char*>(workspace), L,
                    static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------------------------
// The entry point that allocates nothing: the same computation on a file-scope device array.
// Each GPU the library runs on holds its own copy of `scratch` (at its own address) until the
// process ends. Host code never passes the array's name to a kernel or copy (on the host the
// name is a stand-in, not a device address): it uses the address hipGetSymbolAddress returns
// for the current device, looked up once per device and kept.
namespace {

constexpr int64_t kScratchBytes = CM_LMHEAD_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_addr[kMaxDevices];  // device address of `scratch` per device, null until found

// The current device's copy of `scratch`, or an error code.
int scratch_of_current_device(char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* addr = nullptr;
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (addr == nullptr || !cm::aligned(addr, 256)) return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_addr[dev] = static_cast<char*>(addr);
  }
  *out = g_scratch_addr[dev];
  return 0;
}

// The chunk the scratch can hold: chunk_cols itself when given (0 when it does not fit), else
// the largest multiple of 256 columns (at most the whole vocabulary) whose layout fits.
int64_t scratch_chunk(int64_t n_rows, int64_t vocab, int hidden, int64_t chunk_cols,
                      bool want_grad, bool need_wt) {
  auto fits = [&](int64_t c) {
    return layout(n_rows, vocab, hidden, c, want_grad, need_wt).total <= kScratchBytes;
  };
  if (chunk_cols > 0) return fits(chunk_cols) ? chunk_cols : 0;
  int64_t lo = 0, hi = round_up(vocab, kChunkAlign) / kChunkAlign;  // in units of 256 columns
  while (lo < hi) {  // largest fitting multiple; the layout grows with the chunk
    const int64_t mid = (lo + hi + 1) / 2;
    if (fits(mid * kChunkAlign)) lo = mid; else hi = mid - 1;
  }
  return lo * kChunkAlign;
}

}  // namespace

extern "C" int cm_lmhead_ce_noalloc(const void* hidden, int64_t ld_h, const void* weight,
                                    int64_t ld_w, const void* weight_t, const int64_t* target,
                                    int64_t n_rows, int64_t vocab, int hidden_size,
                                    int64_t chunk_cols, float* loss, float* entropy,
                                    int32_t* correct, float* grad, float grad_scale,
                                    void* stream) {
  CM_CHECK_ARG(n_rows >= 0);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(args_ok(hidden, ld_h, weight, ld_w, weight_t, target, n_rows, vocab, hidden_size,
                       chunk_cols, loss, entropy, correct));
  const bool want_grad = grad != nullptr;
  const bool need_wt = want_grad && !weight_t;
  const int64_t chunk = scratch_chunk(n_rows, vocab, hidden_size, chunk_cols, want_grad, need_wt);
  if (chunk == 0) return CM_ERROR_SCRATCH_TOO_SMALL;
  const Layout L = layout(n_rows, vocab, hidden_size, chunk, want_grad, need_wt);
  if (L.total > kScratchBytes) return CM_ERROR_SCRATCH_TOO_SMALL;
  char* ws = nullptr;
  const int st = scratch_of_current_device(&ws);
  if (st) return st;
  return run_lmhead(hidden, ld_h, weight, ld_w, weight_t, target, n_rows, vocab, hidden_size,
                    loss, entropy, correct, grad, grad_scale, ws, L,
                    static_cast<hipStream_t>(stream));
}
