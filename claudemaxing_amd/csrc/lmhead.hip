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
// The full [tokens, vocab] logits never exist: one fp16 chunk of E (at most 128 MiB by default)
// lives in the workspace, in 4 KiB blocks of 32 tokens x 64 columns (Tiled32), so that every K3
// A tile is one contiguous span. Both GEMMs read the weight [V][H] as stored: K1 as a row-major
// operand, K3 as a k-major one (vocabulary = K), whose LDS tiles are transposed into MFMA
// fragments by ds_read_b64_tr_b16.
#include <algorithm>
#include <mutex>
#include <numeric>

#include "common.h"
#include "gemm_lds.h"
#include "softmax_state.h"

namespace {

using cm::gemm::KMajor;
using cm::gemm::floatx16;
using cm::gemm::half8;
using cm::gemm::Tiled32;
using cm::gemm::RowMajor;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPanel = 64;          // columns per panel of the blocked layouts
// Logit given to vocabulary rows past a chunk's last column in K1's epilogue: below every fp16
// value (and finite, so that e^{z - m} z is 0, not NaN).
constexpr float kNoLogit = -3.0e38f;
constexpr float kPScale = 1024.0f;  // P16 = fp16(p * kPScale)
constexpr int kStatThreads = 256;
constexpr int kMaxSplit = 32;      // K-slices of the gradient GEMM (small batches take many)
constexpr int kFinalUnrolled = 8;  // K4 slice counts with their own instantiation
constexpr int kRowsPerBlock = 4;  // K2: token rows (one wavefront each) per workgroup

// Tile configurations: BM, BN, wavefront grid WM x WN, stage depth BK, LDS ring stages, and the
// minimum wavefronts per SIMD for __launch_bounds__ (which caps the registers per wavefront:
// 2 gives 256, 1 gives 512).
constexpr int kBM1 = 256, kBN1 = 256, kWM1 = 2, kWN1 = 4, kBK1 = 64, kST1 = 2, kOcc1 = 2;
constexpr int kThreads1 = kWM1 * kWN1 * cm::kWave;
// K3's tile configurations, one per kind of hidden size (the tile's columns): 256 tokens x 192
// hidden units on 4 x 2 wavefronts of 64 x 96 where the hidden size is a multiple of 192
// (Qwen2.5-1.5B's 1536: 8 tiles per 256 tokens, no partial tile), else 256 x 256 on 2 x 4 of
// 128 x 64 where it is a multiple of 256 (2048, 3584, 5120, 8192), else the first.
template <int BM, int BN, int WM, int WN, int BK, int ST, int OCC>
struct K3Cfg {
  static constexpr int kBM = BM, kBN = BN, kWM = WM, kWN = WN, kBK = BK, kST = ST, kOcc = OCC;
  static constexpr int kThreads = WM * WN * cm::kWave;
  static constexpr int kLds = ST * (BM + BN) * (BK / 8);  // uint4 of the LDS ring
};
using K3Tall = K3Cfg<256, 192, 4, 2, 64, 2, 2>;
using K3Square = K3Cfg<256, 256, 2, 4, 64, 2, 2>;
__host__ __device__ constexpr bool k3_square(int hidden) {
  return hidden % 192 != 0 && hidden % 256 == 0;
}
constexpr int kGroup = kBM1 / kWM1;  // vocabulary columns per partial-statistics group
constexpr int kEpiRows = kGroup / 2;  // group rows one lane of K1's epilogue holds per token
static_assert(kGroup % kPanel == 0, "a statistics group is whole panels");
// K2 holds a row's partials in registers, at most 32 per lane: a chunk has at most 64 * 32
// statistics groups.
constexpr int kMaxRowSlots = 32;
constexpr int64_t kMaxChunk = int64_t{64} * kMaxRowSlots * kGroup;


// Partial statistics of one (token, group): group max, sum e^{z - max}, sum e^{z - max} z, first
// argmax as a vocabulary index (-1 when the group holds no valid column).
struct Partial {
  float max, sum, dot;
  int32_t best;
};

// ---------------------------------------------------------------------------------------------
// K1 epilogue: the tile is Z^T (rows = vocabulary columns of the chunk, cols = tokens). A
// wavefront's rows are one statistics group of kGroup columns, and a lane holds the logits of
// one token. E (layout Tiled32: 32 tokens x 64 columns per 4 KiB block, 8-column chunks inside)
// is written straight from the registers: a lane's entries 4b .. 4b + 3 are rows
// 8b + 4h .. 8b + 4h + 3 of the group (h = the lane's half of the wavefront), so after each pair
// of blocks (b, b + 1) trades halves across the two 32-lane halves (v_permlane32_swap_b32: the first operand's upper 32 lanes swap with the
// second operand's lower 32 lanes) lane l < 32 holds all 8 rows of block b and lane l + 32 those
// of block b + 1. One 16-byte store each, 1 KiB contiguous per wavefront instruction, no LDS
// staging and no barrier.
struct EpiProbs {
  static constexpr int kTN = kBN1 / kWN1 / 32;
  _Float16* e16;        // chunk of E = fp16(e^{z - m_g}), layout Tiled32
  int n_tok;
  int n_voc;            // valid columns of the chunk
  int64_t c0;           // first vocabulary index of the chunk
  Partial* part;        // [n_tok, n_groups]
  int n_groups;
  const int64_t* target;
  _Float16* label_z;    // [n_tok][2][64]: the label group's fp16 logits, lane by lane
  int store;            // write E (the gradient needs it)
  int row_blocks;       // ceil(n_tok / 32), E's 32-token blocks per 64-column panel
  int64_t tgt[kTN];     // targets of the lane's tokens, loaded before the main loop

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
  __device__ __forceinline__ void start(floatx16 (&acc)[TM][TN], int mb, int nb, int lane) {
    cm::gemm::ZeroStart::start<TM, TN>(acc, mb, nb, lane);
  }
  template <int TM, int TN>
  __device__ __forceinline__ void started(floatx16 (&)[TM][TN]) {}

  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb, int lane,
                                        uint4*) {
    static_assert(TM * 32 == kGroup, "a wavefront covers one statistics group");
    const int half_id = lane / 32;
    // accumulator element e of a lane is vocabulary row mb + vrow(e)
    auto vrow = [&](int e) { return (e / 16) * 32 + ((e % 16) / 4) * 8 + half_id * 4 + e % 4; };
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int tok = nb + nt * 32 + lane % 32;
      const bool tok_ok = tok < n_tok;
      // fp16 logits of this lane's token, in place of its accumulators (a separate array of 64
      // values made the epilogue spill); rows past the chunk's last column get kNoLogit, which
      // no fp16 logit reaches and whose e^{z - m} is 0, so the loops below need no validity
      // test per element
#define Z(e) acc[(e) / 16][nt][(e) % 16]
      // A plain conversion (an accumulator, not a product, so there is no multiply for the
      // compiler to fuse it with): it can be computed for every element and selected, where
      // cm::from_f32's register pin made the compiler branch around each conversion. Groups
      // wholly inside the chunk (all but the chunk's last tile; wave-uniform) need no select.
      if (mb + kGroup <= n_voc) {
#pragma unroll
        for (int e = 0; e < TM * 16; ++e) Z(e) = static_cast<float>(static_cast<_Float16>(Z(e)));
      } else {
#pragma unroll
        for (int e = 0; e < TM * 16; ++e)
          Z(e) = mb + vrow(e) < n_voc ? static_cast<float>(static_cast<_Float16>(Z(e))) : kNoLogit;
      }
      // group max and first argmax over both halves of the wavefront (branch-free). In a lane,
      // ascending e is ascending vocabulary row (vrow), so the lane's first argmax is the least e
      // holding the lane's maximum: the maximum as four independent running maxima (no compare-
      // select chain through all 64 values), then the least e equal to it, also four chains.
      // Maxima that are not above kNoLogit (no usable logit) leave best = -1.
      constexpr int kQ = TM * 4;  // values per chain
      float mq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        mq[q] = Z(q * kQ);
#pragma unroll
        for (int e = q * kQ + 1; e < (q + 1) * kQ; ++e) mq[q] = fmaxf(mq[q], Z(e));
      }
      float m = fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]));
      int fq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        fq[q] = -1;
#pragma unroll
        for (int e = (q + 1) * kQ - 1; e >= q * kQ; --e) fq[q] = Z(e) == m ? e : fq[q];
      }
      const int first = fq[0] >= 0 ? fq[0] : fq[1] >= 0 ? fq[1] : fq[2] >= 0 ? fq[2] : fq[3];
      int best = m > kNoLogit && first >= 0 ? mb + vrow(first) : -1;
      if (best < 0) m = kNoLogit;
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
      // e^{z - m_g} = 2^(z log2e - m_g log2e): one fused multiply-add for the argument
      const float mg2 = mg * cm::kLog2e;
      float s = 0.0f, d = 0.0f;
#pragma unroll
      for (int e = 0; e < TM * 16; ++e) {
        // 0 for kNoLogit rows (the argument rounds to -inf), so x z = -0 there
        const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(Z(e), cm::kLog2e, -mg2));
        s += x;
        d += x * Z(e);
        Z(e) = x;
      }
      s += __shfl_xor(s, 32, cm::kWave);
      d += __shfl_xor(d, 32, cm::kWave);
      if (store) {
        // entries 4b .. 4b + 3 = rows 8b + 4h .. 8b + 4h + 3 (vrow(4b) = 8b + 4h)
        auto pack = [&](int e) {  // two fp16 of entries e, e + 1 as one dword
          const half2v v{static_cast<_Float16>(Z(e)), static_cast<_Float16>(Z(e + 1))};
          return __builtin_bit_cast(uint32_t, v);
        };
#pragma unroll
        for (int b = 0; b < TM * 4; b += 2) {
          const auto s0 = __builtin_amdgcn_permlane32_swap(pack(4 * b), pack(4 * b + 4), false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(pack(4 * b + 2), pack(4 * b + 6), false, false);
          // lane l < 32: block b, rows 0-3 (its own) then 4-7; lane l + 32: block b + 1
          const u32x4 chunk{s0[0], s1[0], s0[1], s1[1]};
          const int v = mb + 8 * (b + half_id);  // first vocabulary column (of the chunk)
          // streamed past the caches: K3 reads E only after K1 has finished every tile
          // (1.7% off the call against plain stores, same-process A/B)
          if (tok_ok)
            __builtin_nontemporal_store(
                chunk, reinterpret_cast<u32x4*>(e16 + Tiled32::index(tok, v, row_blocks)));
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
  }
};

// K3 epilogue: the tile is G (rows = tokens, cols = hidden units). On later chunks the
// accumulators start from the slice's previous value times the row's rescale factor: start()
// issues those loads (from clamped addresses, so without branches) ahead of the first stage's
// loads, whose wait they share, and started() applies the factors; apply() then only stores. A
// workgroup thus spends no round trip of its own on the read-modify-write of its slice.
struct EpiGrad {
  static constexpr int kMaxTM = 4;
  float* grad;          // [n_tok, hidden] fp32 accumulator of this K-slice
  int n_tok;
  int hidden;
  const float* factor;  // [n_tok]
  int first;            // first chunk: G = acc
  float f[kMaxTM][16];  // factors of the lane's accumulator rows, loaded by start()

  template <int TM, int TN>
  __device__ __forceinline__ void prepare(int, int, int) {}

  // token row of accumulator entry r of tile row mt, and hidden unit of tile column nt
  static __device__ __forceinline__ int row_of(int mb, int mt, int r, int lane) {
    return mb + mt * 32 + (r / 4) * 8 + (lane / 32) * 4 + (r % 4);
  }
  static __device__ __forceinline__ int col_of(int nb, int nt, int lane) {
    return nb + nt * 32 + lane % 32;
  }

  template <int TM, int TN>
  __device__ __forceinline__ void start(floatx16 (&acc)[TM][TN], int mb, int nb, int lane) {
    static_assert(TM <= kMaxTM, "factor rows of the wavefront tile");
    if (first) {
      cm::gemm::ZeroStart::start<TM, TN>(acc, mb, nb, lane);
      return;
    }
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tok = row_of(mb, mt, r, lane);
        const int64_t row = tok < n_tok ? tok : 0;
        f[mt][r] = factor[row];
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          const int h = col_of(nb, nt, lane);
          acc[mt][nt][r] = grad[row * hidden + (h < hidden ? h : 0)];
        }
      }
  }

  template <int TM, int TN>
  __device__ __forceinline__ void started(floatx16 (&acc)[TM][TN]) {
    if (first) return;
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) acc[mt][nt][r] *= f[mt][r];
  }

  template <int TM, int TN>
  __device__ __forceinline__ void apply(floatx16 (&acc)[TM][TN], int mb, int nb, int lane,
                                        uint4*) const {
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tok = row_of(mb, mt, r, lane);
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          const int h = col_of(nb, nt, lane);
          if (tok < n_tok && h < hidden) grad[static_cast<int64_t>(tok) * hidden + h] = acc[mt][nt][r];
        }
      }
  }
};

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

// K3: each K-slice accumulates into its own buffer.
struct GradSlices {
  float* g[kMaxSplit];
};

// One K1 launch's arguments: Z^T = A B^T with A = the chunk's weight rows, B = the hidden rows.
struct K1Job {
  RowMajor A, B;
  int count;  // workgroups (tiles)
  int remap;  // XCD-aware tile order (count % 8 == 0)
  EpiProbs epi;
};

// One K3 launch's arguments: G_s = G_s * factor + P W_c over K-slices of k_slice columns.
struct K3Job {
  Tiled32 A;  // E
  KMajor B;   // W_c as stored ([C][H], hidden contiguous), read as the operand W_c^T
  int tiles;  // output tiles; count = tiles * n_split workgroups
  int count;
  int k_slice;
  int remap;
  GradSlices out;
  int n_tok, hidden;
  const float* factor;
  int first;
  const float* scale;
};

constexpr int kLds1 = kST1 * (kBM1 + kBN1) * (kBK1 / 8);  // uint4 of K1's LDS ring

__device__ __forceinline__ void k1_block(const K1Job& j, int bid, uint4* lds) {
  int tm, tn;
  cm::gemm::tile_of(bid, j.count, (j.B.rows + kBN1 - 1) / kBN1, j.remap, tm, tn);
  EpiProbs epi = j.epi;
  cm::gemm::gemm_lds<kBM1, kBN1, kWM1, kWN1, kBK1, kST1>(j.A, j.B, 0, j.A.k_len, tm, tn, epi, lds);
}

template <class CFG, int EDGE>
__device__ __forceinline__ void k3_block(const K3Job& j, int bid, uint4* lds) {
  int tm, tn, s;
  cm::gemm::tile_of_sliced(bid, j.count, j.tiles, (j.B.rows + CFG::kBN - 1) / CFG::kBN, j.remap,
                           tm, tn, s);
  const int k_begin = s * j.k_slice;
  // An empty slice still runs the epilogue (with zero accumulators) so that its buffer is
  // initialised on the first chunk and rescaled on later ones.
  const int k_end = max(k_begin, min(j.A.k_len, k_begin + j.k_slice));
  EpiGrad epi{j.out.g[s], j.n_tok, j.hidden, j.factor, j.first, {}};  // f: start()
  using FX = ScaleP<CFG::kBM / CFG::kWM / 32>;
  FX xp{j.scale, j.n_tok, 0, {}, {}};  // nxt / cur are filled by prefetch
  cm::gemm::gemm_lds<CFG::kBM, CFG::kBN, CFG::kWM, CFG::kWN, CFG::kBK, CFG::kST, Tiled32, KMajor,
                     EpiGrad, FX, EDGE>(j.A, j.B, k_begin, k_end, tm, tn, epi, lds, xp);
}

// __launch_bounds__'s second argument is the minimum number of wavefronts per SIMD, which caps
// the registers per wavefront accordingly.
__global__ __launch_bounds__(kThreads1, kOcc1) void lmh_gemm1(K1Job j) {
  __shared__ uint4 lds[kLds1];
  k1_block(j, static_cast<int>(blockIdx.x), lds);
}

// EDGE: cm::gemm::kEdgeNever when every output tile lies inside G (n_tok a multiple of the
// tile's rows, hidden of its columns; the contraction runs over whole 64-column panels), else
// kEdgeAlways. One loop copy per kernel: two in one did not fit the registers.
template <class CFG, int EDGE>
__global__ __launch_bounds__(CFG::kThreads, CFG::kOcc) void lmh_gemm3(K3Job j) {
  __shared__ uint4 lds[CFG::kLds];
  k3_block<CFG, EDGE>(j, static_cast<int>(blockIdx.x), lds);
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

// Merge the states of the 64 lanes of a wavefront; every lane gets the result.
__device__ __forceinline__ OffState wave_merge_off(OffState s) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) {
    OffState o{cm::shfl_xor_state(s.st, d), __shfl_xor(s.off, d, cm::kWave)};
    s.merge(o);
  }
  return s;
}

// K2: merge the chunk's partials into the running state; the factor; with a scale array, the
// group scales s_g = e^{m_g - lse} * 1024 of labelled tokens ([groups][n_tok], 0 otherwise),
// and the label's own entry of E set to 0 when the label falls in this chunk: the label's
// coefficient p_t - 1 is applied by K4 in fp32, so its near-1 probability never enters the
// fp32 accumulators (a ~1024 W_t term there would cancel against -1024 W_t only at the end,
// losing the small difference 1 - p_t of a confident label to the accumulators' rounding).
//
// One wavefront per token row; lane l holds groups l, l + 64, ... (SLOTS of them, the chunk's
// groups being at most 64 * SLOTS). Every load of the row (the running state, the SLOTS
// partials, the label group's logits) is issued before the first merge, so a row costs one
// memory round trip; the group maxima stay in registers for the scales.
template <int SLOTS>
__global__ __launch_bounds__(kRowsPerBlock * cm::kWave) void lmh_rows_kernel(
    const Partial* __restrict__ part, int n_groups, RowState rs,
    const int64_t* __restrict__ target, int n_tok, int64_t c0, int n_voc, int first,
    float* __restrict__ scale, _Float16* __restrict__ e16, const _Float16* __restrict__ label_z,
    int row_blocks) {
  const int lane = threadIdx.x % cm::kWave;
  const int row = blockIdx.x * kRowsPerBlock + static_cast<int>(threadIdx.x / cm::kWave);
  if (row >= n_tok) return;  // the whole wavefront
  const int64_t t = target[row];
  const bool labelled = t != -100;
  // the label's statistics group in this chunk, or -1
  const int64_t g_label = t >= c0 && t < c0 + n_voc ? (t - c0) / kGroup : -1;
  const int n_valid = (n_voc + kGroup - 1) / kGroup;  // groups K1 wrote for this chunk
  OffState now = OffState::empty();
  if (!first) {
    now.st = cm::SoftmaxState{rs.max[row], rs.sum[row], rs.dot[row], rs.best[row]};
    now.off = rs.off[row];
  }
  const uint4* prow = reinterpret_cast<const uint4*>(part + static_cast<int64_t>(row) * n_groups);
  Partial p[SLOTS];
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const int g = lane + i * cm::kWave;
    p[i] = __builtin_bit_cast(Partial, prow[g < n_valid ? g : 0]);
  }
  // The label group's 128 fp16 logits (K1 copied them out lane by lane: entry e of the lane in
  // half h is group row (e/16)*32 + ((e%16)/4)*8 + 4h + e%4); rows past the chunk hold the
  // sentinel logit. They give the label's logit and the group's sum of e^{z - m_g} over its
  // other columns, relative to the group max as K1's sums are.
  float z0 = 0.0f, z1 = 0.0f;
  if (g_label >= 0) {  // uniform over the wavefront
    const _Float16* lz = label_z + static_cast<int64_t>(row) * 2 * kEpiRows;
    z0 = static_cast<float>(lz[lane]);
    z1 = static_cast<float>(lz[kEpiRows + lane]);
  }
  float label_off = 0.0f;
  if (g_label >= 0) {
    const int local = static_cast<int>(t - c0 - g_label * kGroup);
    const int slot = static_cast<int>(g_label / cm::kWave), owner = static_cast<int>(g_label % cm::kWave);
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i)
      if (i == slot) mine = p[i].max;
    const float mg = __shfl(mine, owner, cm::kWave);
    const int r0 = (lane / 16) * 32 + ((lane % 16) / 4) * 8 + lane % 4;  // half 0; half 1: + 4
    const bool has0 = r0 == local, has1 = r0 + 4 == local;
    label_off = cm::wave_sum((has0 ? 0.0f : cm::exp_f(z0 - mg)) + (has1 ? 0.0f : cm::exp_f(z1 - mg)));
    const unsigned long long who = __ballot(has0 || has1);
    const float zt = __shfl(has0 ? z0 : z1, static_cast<int>(__builtin_ctzll(who)), cm::kWave);
    if (lane == 0) rs.label_logit[row] = zt;
  }
  OffState acc = OffState::empty();
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const int g = lane + i * cm::kWave;
    if (g < n_valid && p[i].best >= 0) {
      OffState q{{p[i].max, p[i].sum, p[i].dot, static_cast<int64_t>(p[i].best)},
                 g == g_label ? label_off : p[i].sum};
      acc.merge(q);
    }
  }
  acc = wave_merge_off(acc);
  const float lse_prev = first ? -__builtin_huge_valf() : now.st.lse();
  now.merge(acc);
  const float lse_now = now.st.lse();
  if (lane == 0) {
    rs.max[row] = now.st.max;
    rs.sum[row] = now.st.sum;
    rs.dot[row] = now.st.dot;
    rs.best[row] = static_cast<int32_t>(now.st.best);
    rs.off[row] = now.off;
    rs.lse[row] = lse_now;
    rs.factor[row] = first ? 0.0f : cm::exp_f(lse_prev - lse_now);
  }
  if (scale == nullptr) return;
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const int g = lane + i * cm::kWave;
    if (g < n_valid)
      scale[static_cast<int64_t>(g) * n_tok + row] =
          labelled ? cm::exp_f(p[i].max - lse_now) * kPScale : 0.0f;
  }
  if (lane == 0 && g_label >= 0)
    e16[Tiled32::index(row, t - c0, row_blocks)] = static_cast<_Float16>(0.0f);
}

// K4: final per-row outputs; G = scale * (sum_s G_s / 1024 + (p_t - 1) W[t]) for labelled rows,
// else 0. NS = the number of K-slices; a thread handles kFinalPer hidden units at a time and
// issues all their loads (NS slices and W[t]) before the first store.
constexpr int kFinalPer = 8;

template <int NS>
__global__ __launch_bounds__(kStatThreads) void lmh_final_kernel(
    RowState rs, const int64_t* __restrict__ target, int64_t vocab, float* __restrict__ loss,
    float* __restrict__ entropy, int32_t* __restrict__ correct, GradSlices gs,
    const _Float16* __restrict__ weight, int64_t ld_w, int hidden, float grad_scale, int ns) {
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
  // NS > 0: NS slices, every load issued before the first add; NS == 0: ns slices (more than
  // kFinalUnrolled), loaded kFinalUnrolled at a time. Either way the slices are added in order.
  constexpr int kV = NS > 0 ? NS : kFinalUnrolled;
  for (int h0 = threadIdx.x; h0 < hidden; h0 += kStatThreads * kFinalPer) {
    float v[kV][kFinalPer], wv[kFinalPer], accs[kFinalPer];
#pragma unroll
    for (int j = 0; j < kFinalPer; ++j) {
      const int h = h0 + j * kStatThreads;
      const int hc = h < hidden ? h : 0;
      wv[j] = static_cast<float>(w[hc]);
#pragma unroll
      for (int s = 0; s < kV; ++s) v[s][j] = gs.g[s][off + hc];
    }
#pragma unroll
    for (int j = 0; j < kFinalPer; ++j) {
      accs[j] = v[0][j];
#pragma unroll
      for (int s = 1; s < kV; ++s) accs[j] += v[s][j];
    }
    if constexpr (NS == 0) {
      for (int s0 = kFinalUnrolled; s0 < ns; s0 += kFinalUnrolled) {
#pragma unroll
        for (int j = 0; j < kFinalPer; ++j) {
          const int h = h0 + j * kStatThreads;
          const int hc = h < hidden ? h : 0;
#pragma unroll
          for (int s = 0; s < kFinalUnrolled; ++s)
            v[s][j] = s0 + s < ns ? gs.g[s0 + s][off + hc] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kFinalPer; ++j)
#pragma unroll
          for (int s = 0; s < kFinalUnrolled; ++s)
            if (s0 + s < ns) accs[j] += v[s][j];
      }
    }
#pragma unroll
    for (int j = 0; j < kFinalPer; ++j) {
      const int h = h0 + j * kStatThreads;
      const float acc = accs[j];
      if (h < hidden)
        gs.g[0][off + h] = labelled && in_range
                               ? grad_scale * (acc * (1.0f / kPScale) + coef * wv[j])
                               : (labelled ? __builtin_nanf("") : 0.0f);
    }
  }
}

// K4 for n_split slices (1 <= n_split <= kMaxSplit).
int launch_final(int n_split, int n_tok, hipStream_t s, const RowState& rs, const int64_t* target,
                 int64_t vocab, float* loss, float* entropy, int32_t* correct, const GradSlices& gs,
                 const _Float16* w, int64_t ld_w, int hidden, float grad_scale) {
#define CM_FINAL(NS)                                                                            \
  hipLaunchKernelGGL(lmh_final_kernel<NS>, dim3(n_tok), dim3(kStatThreads), 0, s, rs, target,    \
                     vocab, loss, entropy, correct, gs, w, ld_w, hidden, grad_scale, n_split)
  if (n_split > kFinalUnrolled && n_split <= kMaxSplit) {
    CM_FINAL(0);
    return cm::launch_status();
  }
  switch (n_split) {
    case 1: CM_FINAL(1); break;
    case 2: CM_FINAL(2); break;
    case 3: CM_FINAL(3); break;
    case 4: CM_FINAL(4); break;
    case 5: CM_FINAL(5); break;
    case 6: CM_FINAL(6); break;
    case 7: CM_FINAL(7); break;
    case 8: CM_FINAL(8); break;
    default: return static_cast<int>(hipErrorInvalidValue);
  }
#undef CM_FINAL
  return cm::launch_status();
}

// ---------------------------------------------------------------------------------------------
// Workspace layout.
int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

constexpr int64_t kChunkAlign = kBM1 > 256 ? kBM1 : 256;
constexpr int64_t kCUs = 256;  // MI355X compute units (8 XCDs x 32)

// E's token rows: padded to the gradient GEMM's 256-row tiles, so that its loads of a partial
// tile stay inside E and need no bounds selection (the padding rows feed only output rows that
// are never stored).
constexpr int64_t kERowAlign = 256;
static_assert(K3Tall::kBM == kERowAlign && K3Square::kBM == kERowAlign,
              "a K3 tile's rows are one padded block of E rows");
int64_t e_rows(int64_t n_rows) { return round_up(n_rows > 0 ? n_rows : 1, kERowAlign); }
int e_row_blocks(int64_t n_rows) { return static_cast<int>(e_rows(n_rows) / 32); }

int64_t default_chunk(int64_t n_rows, int64_t vocab) {
  // E chunk of at most 128 MiB (fp16, padded rows x C). Per extra chunk the gradient GEMM's
  // split-K slices are read and rewritten once more (4 x 12.6 MB at N = 2048) and each kernel
  // ramps up once more. K1 runs one 256 x 256 workgroup per CU, so the chunk is chosen by the
  // waves of workgroups the whole vocabulary takes: the number of 256-column vocabulary tiles
  // per chunk (from the budget down to half of it) that needs the fewest waves over all chunks,
  // then the fewest chunks. At N = 2048 (8 token tiles) that is 4 chunks of 128 tiles (32768
  // columns, 1024 workgroups each) and the rest, 19 waves; at 1792 (7 token tiles) 4 chunks of
  // 146 tiles (1022 workgroups) and the rest, 17 waves where equal chunks of 119 took 20.
  // Measured at N = 2048, V = 151936 (one MI355X, one process, interleaved): 4 x 32768 + 20864
  // columns 2092 us, 5 x 30464 2105 us, 24576 2115 us, 16384 2171 us.
  const int64_t budget = (int64_t{128} << 20) / 2 / e_rows(n_rows);  // columns
  int64_t c = budget / kChunkAlign * kChunkAlign;
  if (c < 4096) c = 4096;
  if (c > kMaxChunk) c = kMaxChunk;
  if (c >= vocab) return round_up(vocab, kChunkAlign);
  const int64_t token_tiles = (n_rows + kBN1 - 1) / kBN1;
  const int64_t vocab_tiles = (vocab + kBM1 - 1) / kBM1;
  auto waves = [&](int64_t tiles) { return (tiles * token_tiles + kCUs - 1) / kCUs; };
  int64_t best_vt = c / kBM1, best_waves = -1, best_chunks = 0;
  for (int64_t vt = c / kBM1; vt >= 1 && vt * 2 >= c / kBM1; --vt) {
    const int64_t full = vocab_tiles / vt, rest = vocab_tiles % vt;
    const int64_t w = full * waves(vt) + (rest ? waves(rest) : 0);
    const int64_t n = full + (rest ? 1 : 0);
    if (best_waves < 0 || w < best_waves || (w == best_waves && n < best_chunks)) {
      best_vt = vt;
      best_waves = w;
      best_chunks = n;
    }
  }
  return best_vt * kBM1;
}

// Output tiles of the gradient GEMM (K3) for this hidden size's tile configuration.
int64_t k3_tiles(int64_t n_rows, int hidden) {
  const int bm = k3_square(hidden) ? K3Square::kBM : K3Tall::kBM;
  const int bn = k3_square(hidden) ? K3Square::kBN : K3Tall::kBN;
  return ((n_rows + bm - 1) / bm) * ((hidden + bn - 1) / bn);
}

// K-slices of the gradient GEMM: the grid of tiles x slices should fill whole waves of the 256
// CUs (one workgroup each), but every slice is one more fp32 accumulator to read and rewrite
// per chunk. Take the fewest slices whose wave fill is within 7% of the best one up to
// kMaxSplit (N = 2048: 64 tiles x 4 at hidden 1536, 112 x 2 at 3584, 160 x 3 at 5120; N = 256:
// 8 x 30), among the counts that leave no slice of a full chunk empty (whole_slices: an empty
// slice's accumulator would still be read, rescaled and written back on every chunk, and its
// workgroups would only pad the wave count).
// Slices that hold columns when `groups` statistics groups are split into `sp` slices of equal
// whole-group width (the last one shorter): fewer than sp when the width rounds up.
int64_t whole_slices(int64_t groups, int64_t sp) {
  if (groups <= 0 || sp <= 1) return 1;
  const int64_t width = (groups + sp - 1) / sp;
  return (groups + width - 1) / width;
}

int n_split_for(int64_t n_rows, int hidden, int64_t groups) {
  const int64_t tiles = k3_tiles(n_rows, hidden);
  auto fill = [&](int64_t sp) {
    const int64_t wg = tiles * sp;
    return static_cast<double>(wg) / static_cast<double>((wg + kCUs - 1) / kCUs * kCUs);
  };
  // the extra slices' accumulators within 128 MiB (a small batch can afford many: 1.5 MB each
  // at 256 tokens x 1536)
  const int64_t slice_bytes = round_up(n_rows * hidden * 4, 256);
  int64_t cap = 1 + (int64_t{128} << 20) / (slice_bytes > 0 ? slice_bytes : 1);
  if (cap > kMaxSplit) cap = kMaxSplit;
  auto usable = [&](int sp) { return whole_slices(groups, sp) == sp; };
  double best = 0.0;
  for (int sp = 1; sp <= cap; ++sp)
    if (usable(sp)) best = fill(sp) > best ? fill(sp) : best;
  for (int sp = 1; sp <= cap; ++sp)
    if (usable(sp) && fill(sp) >= best - 0.07) return sp;
  return 1;
}

struct Layout {
  int64_t chunk, n_groups, n_chunks;
  int n_split;
  int64_t off_e16, off_part, off_rows, off_labz, off_scale, off_g, total;
};

Layout layout(int64_t n_rows, int64_t vocab, int hidden, int64_t chunk, bool want_grad,
              int max_split = kMaxSplit) {
  Layout L;
  L.chunk = chunk > 0 ? round_up(chunk, kChunkAlign) : default_chunk(n_rows, vocab);
  if (L.chunk > round_up(vocab, kChunkAlign)) L.chunk = round_up(vocab, kChunkAlign);
  if (L.chunk > kMaxChunk) L.chunk = kMaxChunk;
  L.n_groups = L.chunk / kGroup;
  L.n_chunks = (vocab + L.chunk - 1) / L.chunk;
  L.n_split = want_grad ? static_cast<int>(whole_slices(
                              L.n_groups, std::min(n_split_for(n_rows, hidden, L.n_groups),
                                                   max_split)))
                        : 1;
  int64_t off = 0;
  L.off_e16 = off;
  off += round_up(e_rows(n_rows) * L.chunk * 2, 256);
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
  L.total = off;
  return L;
}

}  // namespace

extern "C" int64_t cm_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab, int hidden_size,
                                                int64_t chunk_cols) {
  if (n_rows <= 0 || vocab <= 0 || hidden_size <= 0) return 0;
  return layout(n_rows, vocab, hidden_size, chunk_cols, true).total;
}

extern "C" int cm_lmhead_ce_plan(int64_t n_rows, int64_t vocab, int hidden_size,
                                 int64_t chunk_cols, int64_t* chunk, int* n_split) {
  CM_CHECK_ARG(n_rows > 0 && vocab > 0 && hidden_size > 0 && chunk_cols >= 0);
  CM_CHECK_ARG(chunk != nullptr && n_split != nullptr);
  const Layout L = layout(n_rows, vocab, hidden_size, chunk_cols, true);
  *chunk = L.chunk;
  *n_split = L.n_split;
  return 0;
}

namespace {

// Argument checks shared by both entry points (everything but the workspace).
bool args_ok(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
             const int64_t* target, int64_t n_rows, int64_t vocab,
             int hidden_size, int64_t chunk_cols, const float* loss, const float* entropy,
             const int32_t* correct) {
  if (!(n_rows > 0 && vocab > 0 && hidden_size > 0 && chunk_cols >= 0)) return false;
  if (!(hidden && weight && target && loss && entropy && correct)) return false;
  if (!(n_rows < (int64_t{1} << 31) && vocab < (int64_t{1} << 31))) return false;
  // 16-byte tile rows: hidden size, leading dimensions and bases multiples of 8 fp16.
  return hidden_size % 8 == 0 && ld_h % 8 == 0 && ld_w % 8 == 0 && ld_h >= hidden_size &&
         ld_w >= hidden_size && cm::aligned(hidden, 16) && cm::aligned(weight, 16);
}

// The launches of one call (K1..K4 per chunk), on `ws` laid out as L; the arguments and the
// workspace's size and alignment have been checked.
int run_lmhead(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
               const int64_t* target, int64_t n_rows, int64_t vocab,
               int hidden_size, float* loss, float* entropy, int32_t* correct, float* grad,
               float grad_scale, char* ws, const Layout& L, hipStream_t s) {
  const bool want_grad = grad != nullptr;
  Partial* part = reinterpret_cast<Partial*>(ws + L.off_part);
  float* scale = want_grad ? reinterpret_cast<float*>(ws + L.off_scale) : nullptr;
  const RowState rs = row_state(ws + L.off_rows, round_up(n_rows * 4, 256));
  if (!complete(rs)) return static_cast<int>(hipErrorInvalidValue);
  _Float16* label_z = reinterpret_cast<_Float16*>(ws + L.off_labz);
  GradSlices gs{};
  gs.g[0] = grad;
  for (int i = 1; i < L.n_split; ++i)
    gs.g[i] = reinterpret_cast<float*>(ws + L.off_g + (i - 1) * round_up(n_rows * hidden_size * 4, 256));
  const _Float16* H16 = static_cast<const _Float16*>(hidden);
  const _Float16* W16 = static_cast<const _Float16*>(weight);
  const int n_tok = static_cast<int>(n_rows);

  auto c0_of = [&](int64_t c) { return c * L.chunk; };
  auto n_voc_of = [&](int64_t c) {
    return static_cast<int>(vocab - c0_of(c) < L.chunk ? vocab - c0_of(c) : L.chunk);
  };
  _Float16* e16 = reinterpret_cast<_Float16*>(ws + L.off_e16);
  auto e16_of = [&](int64_t) { return e16; };
  // K1 of chunk c: Z^T tile = W_c H^T, statistics, E and the label logit
  auto k1_job = [&](int64_t c) {
    const int n_voc = n_voc_of(c);
    const int tiles = ((n_voc + kBM1 - 1) / kBM1) * ((n_tok + kBN1 - 1) / kBN1);
    K1Job j{RowMajor{W16 + c0_of(c) * ld_w, ld_w, n_voc, hidden_size},
            RowMajor{H16, ld_h, n_tok, hidden_size},
            tiles,
            tiles % 8 == 0 ? 1 : 0,
            EpiProbs{e16_of(c), n_tok, n_voc, c0_of(c), part, static_cast<int>(L.n_groups), target,
                     label_z, want_grad ? 1 : 0, e_row_blocks(n_tok), {}}};  // tgt: prepare()
    return j;
  };
  // K2 of chunk c: running statistics and the group scales
  auto k2 = [&](int64_t c) {
    const dim3 grid((n_tok + kRowsPerBlock - 1) / kRowsPerBlock), block(kRowsPerBlock * cm::kWave);
    const int ng = static_cast<int>(L.n_groups), fi = c == 0 ? 1 : 0, nv = n_voc_of(c);
    const int64_t c0 = c0_of(c);
    _Float16* e = e16_of(c);
    const int rb = e_row_blocks(n_tok);
    if (L.n_groups <= cm::kWave) {
      hipLaunchKernelGGL(lmh_rows_kernel<1>, grid, block, 0, s, part, ng, rs, target, n_tok, c0,
                         nv, fi, scale, e, label_z, rb);
    } else if (L.n_groups <= 4 * cm::kWave) {
      hipLaunchKernelGGL(lmh_rows_kernel<4>, grid, block, 0, s, part, ng, rs, target, n_tok, c0,
                         nv, fi, scale, e, label_z, rb);
    } else {
      hipLaunchKernelGGL(lmh_rows_kernel<kMaxRowSlots>, grid, block, 0, s, part, ng, rs, target,
                         n_tok, c0, nv, fi, scale, e, label_z, rb);
    }
    return cm::launch_status();
  };
  // K3 of chunk c: G_s = G_s * factor + P W_c over K-slices; B = W_c read as stored (k-major)
  auto k3_job = [&](int64_t c) {
    const int n_voc = n_voc_of(c);
    const int tiles = static_cast<int>(k3_tiles(n_tok, hidden_size));
    const int panels = (n_voc + kPanel - 1) / kPanel;
    // slices are whole statistics groups, so a stage never straddles two group scales
    const int groups = (panels * kPanel + kGroup - 1) / kGroup;
    const int k_slice = ((groups + L.n_split - 1) / L.n_split) * kGroup;
    const int count = tiles * L.n_split;
    K3Job j{Tiled32{e16_of(c), n_tok, n_voc, e_row_blocks(n_tok)},
            KMajor{W16 + c0_of(c) * ld_w, ld_w, hidden_size, n_voc},
            tiles,
            count,
            k_slice,
            count % 8 == 0 ? 1 : 0,
            gs,
            n_tok,
            hidden_size,
            rs.factor,
            c == 0 ? 1 : 0,
            scale};
    return j;
  };

  // per chunk: K1, K2, and with the gradient K3
  for (int64_t c = 0; c < L.n_chunks; ++c) {
    const K1Job j1 = k1_job(c);
    hipLaunchKernelGGL(lmh_gemm1, dim3(j1.count), dim3(kThreads1), 0, s, j1);
    int st = cm::launch_status();
    if (st) return st;
    st = k2(c);
    if (st) return st;
    if (!want_grad) continue;
    const K3Job j3 = k3_job(c);
    auto launch3 = [&](auto cfg) {
      using CFG = decltype(cfg);
      // E's rows are padded to whole tiles (kERowAlign), so only the hidden size and the
      // chunk's columns decide whether every load lies inside its operand
      if (hidden_size % CFG::kBN == 0 && j3.A.k_len % CFG::kBK == 0) {
        hipLaunchKernelGGL((lmh_gemm3<CFG, cm::gemm::kEdgeNever>), dim3(j3.count),
                           dim3(CFG::kThreads), 0, s, j3);
      } else {
        hipLaunchKernelGGL((lmh_gemm3<CFG, cm::gemm::kEdgeAlways>), dim3(j3.count),
                           dim3(CFG::kThreads), 0, s, j3);
      }
    };
    if (k3_square(hidden_size)) {
      launch3(K3Square{});
    } else {
      launch3(K3Tall{});
    }
    st = cm::launch_status();
    if (st) return st;
  }
  GradSlices fin = want_grad ? gs : GradSlices{};
  return launch_final(want_grad ? L.n_split : 1, n_tok, s, rs, target, vocab, loss, entropy,
                      correct, fin, W16, ld_w, hidden_size, grad_scale);
}

}  // namespace

extern "C" int cm_lmhead_ce(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
                            const int64_t* target, int64_t n_rows,
                            int64_t vocab, int hidden_size, int64_t chunk_cols, float* loss,
                            float* entropy, int32_t* correct, float* grad, float grad_scale,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  CM_CHECK_ARG(n_rows >= 0);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(args_ok(hidden, ld_h, weight, ld_w, target, n_rows, vocab, hidden_size,
                       chunk_cols, loss, entropy, correct));
  CM_CHECK_ARG(workspace != nullptr);
  const bool want_grad = grad != nullptr;
  const Layout L = layout(n_rows, vocab, hidden_size, chunk_cols, want_grad);
  CM_CHECK_ARG(workspace_bytes >= L.total && cm::aligned(workspace, 256));
  return run_lmhead(hidden, ld_h, weight, ld_w, target, n_rows, vocab, hidden_size,
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

// Estimated time of one call with layout L, to rank the layouts that fit the scratch. Per
// chunk: the logits GEMM's whole waves of 256 x 256 workgroups (one per CU, ~53 us per wave at
// hidden 1536 on MI355X, epilogue included), the gradient GEMM's work spread over whole waves of
// its tiles x slices (~0.95 PFLOP/s when the grid fills the chip), the read and rewrite of every
// slice's accumulator (~9 TB/s) and ~2 us of launch ramps. At N = 2048 it gives 2090 us for the
// default layout (4 x 32768 + 20864 columns, 4 slices; measured 2094-2124) and 2590 us for
// 23 x 6400 + 4736 columns with 4 slices (measured 2591).
double est_cost_us(int64_t n_rows, int64_t vocab, int hidden, const Layout& L) {
  const int64_t token_tiles = (n_rows + kBN1 - 1) / kBN1;
  const double wave1_us = 53.0 * hidden / 1536.0;
  const int64_t wg3 = k3_tiles(n_rows, hidden) * L.n_split;
  const double fill3 = static_cast<double>(wg3) / static_cast<double>((wg3 + kCUs - 1) / kCUs * kCUs);
  const double rmw_us = 2.0 * L.n_split * static_cast<double>(n_rows) * hidden * 4 / 9.0e6;
  double us = 0.0;
  for (int64_t c = 0; c < L.n_chunks; ++c) {
    const int64_t cols = std::min(L.chunk, vocab - c * L.chunk);
    const int64_t wg1 = (cols + kBM1 - 1) / kBM1 * token_tiles;
    us += static_cast<double>((wg1 + kCUs - 1) / kCUs) * wave1_us;
    us += 2.0 * static_cast<double>(n_rows) * cols * hidden / 0.95e9 / fill3;
    us += (c == 0 ? 0.5 : 1.0) * rmw_us + 2.0;
  }
  return us;
}

// The chunk the scratch can hold: chunk_cols itself when given (0 when it does not fit), else
// the largest multiple of 256 columns (at most the whole vocabulary) whose layout fits.
int64_t scratch_chunk(int64_t n_rows, int64_t vocab, int hidden, int64_t chunk_cols,
                      bool want_grad, int max_split) {
  auto fits = [&](int64_t c) {
    return layout(n_rows, vocab, hidden, c, want_grad, max_split).total <= kScratchBytes;
  };
  if (chunk_cols > 0) return fits(chunk_cols) ? chunk_cols : 0;
  int64_t lo = 0, hi = round_up(vocab, kChunkAlign) / kChunkAlign;  // in units of 256 columns
  while (lo < hi) {  // largest fitting multiple; the layout grows with the chunk
    const int64_t mid = (lo + hi + 1) / 2;
    if (fits(mid * kChunkAlign)) lo = mid; else hi = mid - 1;
  }
  return lo * kChunkAlign;
}

// The layout cm_lmhead_ce_noalloc runs in its scratch (false: none fits). K-slices (each an fp32
// [n_rows, hidden] accumulator) and chunk: with chunk_cols given, the most slices up to the
// workspace entry's that fit beside that chunk; else, of the pairs (slice count, a chunk from
// the largest that fits beside that many slices down to half of it), the one estimated fastest.
bool scratch_layout(int64_t n_rows, int64_t vocab, int hidden, int64_t chunk_cols,
                    bool want_grad, Layout* out) {
  int best_split = 0;
  int64_t best_chunk = 0;
  double best_cost = 0.0;
  for (int sp = kMaxSplit; sp >= 1; --sp) {
    const int64_t largest = scratch_chunk(n_rows, vocab, hidden, chunk_cols, want_grad, sp);
    if (largest == 0) continue;
    // with chunk_cols given, that chunk; else every multiple of 256 columns from the largest
    // that fits down to half of it (a smaller chunk can fill the logits GEMM's waves better)
    const int64_t smallest = chunk_cols > 0 ? largest : std::max<int64_t>(kChunkAlign, largest / 2);
    bool any = false;
    for (int64_t chunk = largest; chunk >= smallest; chunk -= kChunkAlign) {
      const Layout T = layout(n_rows, vocab, hidden, chunk, want_grad, sp);
      if (T.n_split < sp) continue;  // the same layout as a smaller count, visited later
      any = true;
      const double cost = est_cost_us(n_rows, vocab, hidden, T);
      if (best_split == 0 || cost < best_cost) {
        best_split = sp;
        best_chunk = chunk;
        best_cost = cost;
      }
    }
    if (chunk_cols > 0 && any) break;
  }
  if (best_split == 0) return false;
  *out = layout(n_rows, vocab, hidden, best_chunk, want_grad, best_split);
  return out->total <= kScratchBytes;
}

}  // namespace

extern "C" int cm_lmhead_ce_noalloc_plan(int64_t n_rows, int64_t vocab, int hidden_size,
                                         int64_t chunk_cols, int want_grad, int64_t* chunk,
                                         int* n_split) {
  CM_CHECK_ARG(n_rows > 0 && vocab > 0 && hidden_size > 0 && chunk_cols >= 0);
  CM_CHECK_ARG(chunk != nullptr && n_split != nullptr);
  Layout L;
  if (!scratch_layout(n_rows, vocab, hidden_size, chunk_cols, want_grad != 0, &L))
    return CM_ERROR_SCRATCH_TOO_SMALL;
  *chunk = L.chunk;
  *n_split = L.n_split;
  return 0;
}

extern "C" int cm_lmhead_ce_noalloc(const void* hidden, int64_t ld_h, const void* weight,
                                    int64_t ld_w, const int64_t* target,
                                    int64_t n_rows, int64_t vocab, int hidden_size,
                                    int64_t chunk_cols, float* loss, float* entropy,
                                    int32_t* correct, float* grad, float grad_scale,
                                    void* stream) {
  CM_CHECK_ARG(n_rows >= 0);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(args_ok(hidden, ld_h, weight, ld_w, target, n_rows, vocab, hidden_size,
                       chunk_cols, loss, entropy, correct));
  Layout L;
  if (!scratch_layout(n_rows, vocab, hidden_size, chunk_cols, grad != nullptr, &L))
    return CM_ERROR_SCRATCH_TOO_SMALL;
  char* ws = nullptr;
  const int st = scratch_of_current_device(&ws);
  if (st) return st;
  return run_lmhead(hidden, ld_h, weight, ld_w, target, n_rows, vocab, hidden_size,
                    loss, entropy, correct, grad, grad_scale, ws, L,
                    static_cast<hipStream_t>(stream));
}
