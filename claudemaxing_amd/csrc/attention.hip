// Causal grouped-query attention over a packed batch of variable-length rows (gfx950):
// forward, and backward as dQ / dK+dV passes, on v_mfma_f32_32x32x16_f16 with fp32
// accumulation and fp32 softmax statistics.
//
// Replaces, for the packed batch of the fused training forward, what transformers' sdpa
// attention computes from the packed block-diagonal causal mask (the reference builds that mask
// in lm_head_loss.py:332-336 and hands it to grouped SDPA, attention.py:332-373): every query at
// row position t attends the keys of its own row at positions 0..t. Here no mask exists: the
// row bounds are kernel arguments, and only the blocks on or below each row's diagonal are
// visited.
//
// Layout. Rows are laid out "row-aligned" in a padded position space: row r starts at position
// pstart[r] = sum over earlier rows of round_up(len, 64), so every 64-token block of a row
// starts 64-aligned and the MFMA operand tiles are whole 16-byte chunks. A relayout pass writes
// fp16 copies of the operands in that space, zero in the pad slots:
//   natural    X16[head][pos][d]                      (d contiguous)
//   transposed XT16[head][d][pos] with the positions of every 16-group stored in the order
//              0-3, 8-11, 4-7, 12-15 (bits 2 and 3 of the position swapped).
// The order is the one in which a lane of a 32x32 MFMA accumulator holds its 16 rows: lane l
// holds rows (e/4)*8 + (l/32)*4 + e%4, so accumulator elements 8j..8j+7 are, in that order, the 8
// operand slots of k-step j for half l/32. A probability tile computed as an accumulator thus
// feeds the next MFMA straight from registers, against a transposed operand tile read as one
// 16-byte chunk per lane.
//
// The row bounds are a device-resident image (Rows, written by cm_attn_rows_image on the host and
// copied to the device by the caller) and the grids are sized for a capacity of padded positions
// given by the caller: blocks past the image's own padded count exit at once. One launch, or one
// captured HIP graph, thus serves every packing whose padded count fits the capacity, the image
// being rewritten before each replay. Every kernel checks the image against the capacity and the
// token count it was launched for, and a workgroup whose row is inconsistent writes nothing.
//
// Forward, per (64-query block, head): S^T = K Q^T (lane = query, so the row statistics are
// lane-local up to one shuffle between the two lane halves), online softmax in the log2 domain,
// O^T += V^T P^T. The log2-domain log-sum-exp of every position is kept for the backward.
// Backward: Delta = rowsum(dO * O); per (64-key block, query head) S = Q K^T and dP = dO V^T,
// P = exp2(S*c - lse2), dS = P (dP - Delta), dV^T += dO^T P, dK^T += Q^T dS, written as per-head
// partials and summed over the heads of each key/value group by a last pass (no atomics: the
// results are the same bits on every run); per (64-query block, head) S^T and dP^T again and
// dQ^T += K^T dS^T.
#include <cstring>

#include "common.h"
#include "gemm_lds.h"

namespace {

using cm::gemm::floatx16;
using cm::gemm::half8;

constexpr int kD = 128;       // head dimension
constexpr int kBlk = 64;      // tokens per block (rows are padded to multiples of it)
constexpr int kMaxRows = 128; // rows of one packed batch
constexpr int kThreads = 256; // two pairs of wavefronts of 32 queries (or keys) each
constexpr int kPairThreads = 128;

struct Rows {
  int start[kMaxRows + 1];   // first real token of row r; start[n] = number of tokens
  int pstart[kMaxRows + 1];  // first padded position of row r (multiples of kBlk)
  int n;
};

// Row holding padded block b (pstart[r] / kBlk <= b < pstart[r + 1] / kBlk).
__device__ __forceinline__ int row_of_block(const Rows& rows, int b) {
  int r = 0;
  while (r + 1 < rows.n && rows.pstart[r + 1] / kBlk <= b) ++r;
  return r;
}

// Whether padded block b of a launch for n_tokens tokens and n_pad padded positions has work:
// the image is consistent with the launch (a row count the struct holds, n_tokens tokens, a
// padded count within n_pad) and b lies inside its padded positions, in a row whose real tokens
// fit its padded blocks. Uniform over the workgroup (scalar loads of the image).
__device__ __forceinline__ bool block_live(const Rows& rows, int b, int n_tokens, int n_pad) {
  const int n = rows.n;
  if (n < 1 || n > kMaxRows || rows.start[n] != n_tokens || rows.pstart[n] > n_pad ||
      b * kBlk >= rows.pstart[n])
    return false;
  const int r = row_of_block(rows, b);
  const int len = rows.start[r + 1] - rows.start[r];
  return len >= 0 && rows.start[r] >= 0 && len <= rows.pstart[r + 1] - rows.pstart[r] &&
         rows.pstart[r] % kBlk == 0 && rows.start[r + 1] <= n_tokens;
}

// Where padded block b lies: its row r, the row's first real token, real length and first padded
// position; live = false for a block with no work (block_live).
struct Where {
  bool live;
  int r, start, len, pstart;
};

// block_live and row_of_block in one round of loads: lane i of the wavefront loads start[i] and
// pstart[i] (one coalesced load each) beside the scalar load of the row count, the block's row
// is the number of rows 1 .. n - 1 that start at or before it (a ballot: pstart is
// non-decreasing, so they are a prefix), and the entries the block needs are read from the lanes
// that hold them. The walk over pstart loaded one entry after the other, a dependent load per row
// at the start of every workgroup. Batches of 64 rows or more take the walk. Called with every
// lane of the wavefront active and b uniform.
__device__ __forceinline__ Where locate(const Rows& rows, int b, int n_tokens, int n_pad) {
  const int n = rows.n;
  const int lane = threadIdx.x % cm::kWave;
  const int stv = rows.start[lane], psv = rows.pstart[lane];  // lane <= 63 < kMaxRows + 1
  Where w{false, 0, 0, 0, 0};
  if (n < 1 || n >= cm::kWave) {
    if (!block_live(rows, b, n_tokens, n_pad)) return w;
    w.r = row_of_block(rows, b);
    w.start = rows.start[w.r];
    w.len = rows.start[w.r + 1] - w.start;
    w.pstart = rows.pstart[w.r];
    w.live = true;
    return w;
  }
  const int pend = __builtin_amdgcn_readlane(psv, n);
  if (__builtin_amdgcn_readlane(stv, n) != n_tokens || pend > n_pad || b * kBlk >= pend)
    return w;
  const int r = __popcll(__ballot(lane >= 1 && lane < n && psv / kBlk <= b));
  const int s0 = __builtin_amdgcn_readlane(stv, r), s1 = __builtin_amdgcn_readlane(stv, r + 1);
  const int p0 = __builtin_amdgcn_readlane(psv, r), p1 = __builtin_amdgcn_readlane(psv, r + 1);
  w.len = s1 - s0;
  w.live = w.len >= 0 && s0 >= 0 && w.len <= p1 - p0 && p0 % kBlk == 0 && s1 <= n_tokens;
  w.r = r;
  w.start = s0;
  w.pstart = p0;
  return w;
}

// Grids of the forward and backward kernels: (heads, padded blocks), heads the fast dimension,
// so that the blocks of one position are dispatched together. A query block's work grows with
// its index in its row (it sees every key block before it), so the query kernels take the
// padded blocks in reverse: the last (heaviest) blocks of the rows go out first and the ones
// that wait for a free CU when the blocks outnumber the CUs (264 at the training step's 1276
// tokens) are rows' first, lightest blocks. The key-block kernel's work shrinks along a row, so
// it keeps the natural order.
__device__ __forceinline__ int heavy_first_query_block() {
  return static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y);
}

// Stored slot of position p inside its 16-group (an involution: bits 2 and 3 swapped).
__device__ __forceinline__ int perm16(int p) {
  return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1);
}

__device__ __forceinline__ floatx16 mfma(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Accumulator elements 8j..8j+7 as the fp16 operand of k-step j.
__device__ __forceinline__ half8 frag_of(const floatx16& a, int j) {
  half8 f;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = static_cast<_Float16>(a[8 * j + i]);
  return f;
}

// Eight consecutive elements of a (fp32 or fp16) tensor as fp16 (round to nearest even).
__device__ __forceinline__ half8 load8(const void* base, int dtype, int64_t off) {
  half8 f;
  if (dtype == CM_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    const float4 a = p[0], b = p[1];
    f[0] = static_cast<_Float16>(a.x); f[1] = static_cast<_Float16>(a.y);
    f[2] = static_cast<_Float16>(a.z); f[3] = static_cast<_Float16>(a.w);
    f[4] = static_cast<_Float16>(b.x); f[5] = static_cast<_Float16>(b.y);
    f[6] = static_cast<_Float16>(b.z); f[7] = static_cast<_Float16>(b.w);
  } else {
    f = *reinterpret_cast<const half8*>(static_cast<const _Float16*>(base) + off);
  }
  return f;
}

__device__ __forceinline__ half8 zero8() {
  half8 f;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = static_cast<_Float16>(0.0f);
  return f;
}

// Eight consecutive elements of a (fp32 or fp16) tensor as fp32.
__device__ __forceinline__ void load8f(const void* base, int dtype, int64_t off, float (&f)[8]) {
  if (dtype == CM_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    const float4 a = p[0], b = p[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const half8 h = *reinterpret_cast<const half8*>(static_cast<const _Float16*>(base) + off);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = static_cast<float>(h[i]);
  }
}

// Qwen2's rotary embedding fused into the attention: the rotation of the forward's q and k and
// of the backward's q and k, and the transposed rotation of the gradients dq and dk. cos / sin
// are fp32 rows [N][D] of the packed tokens with row stride cs_t; cos == nullptr: no rotation.
struct Rope {
  const float* cos;
  const float* sin;
  int64_t cs_t;
};

// One element of the rotation, with h = D / 2: the forward writes o[d] = x[d] c[d] - x[d+h] s[d]
// and o[d+h] = x[d+h] c[d+h] + x[d] s[d+h]; the gradient's transposed rotation writes
// o[d] = g[d] c[d] + g[d+h] s[d+h] and o[d+h] = g[d+h] c[d+h] - g[d] s[d]. x is the element, p
// its partner (d +- h), cs the element's cos and sn the sin the formula takes (the element's
// forward, the partner's backward). Each product is rounded before the sum, as the separate RoPE
// kernel (no contraction) rounds them: the fused rotation gives its bits.
__device__ __forceinline__ float rot_minus(float x, float p, float cs, float sn) {
#pragma clang fp contract(off)
  return x * cs - p * sn;
}
__device__ __forceinline__ float rot_plus(float x, float p, float cs, float sn) {
#pragma clang fp contract(off)
  return x * cs + p * sn;
}

// LDS tiles filled by global_load_lds_dwordx4 (64 lanes x 16 bytes into 64 consecutive slots).
// A tile has ROWS rows of CH 16-byte chunks; the chunk of (row, logical c) is stored at
// physical chunk c ^ swz(row), chosen so that a fragment read (16 consecutive rows at one
// logical chunk per 16 lanes) hits 16 distinct bank groups:
//   CH = 16 (256-byte rows): row & 15;  CH = 8: (row >> 1) & 7;  CH = 4: (row >> 2) & 3.
template <int CH>
__device__ __forceinline__ int swz(int row) {
  return CH == 16 ? (row & 15) : CH == 8 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

template <int CH>
__device__ __forceinline__ half8 frag(const uint4* tile, int row, int c) {
  return __builtin_bit_cast(half8, tile[row * CH + (c ^ swz<CH>(row))]);
}

// Issue this thread's loads of a ROWS x CH tile whose row i starts at src + i * row_bytes; the
// two wavefronts of a pair (wave = 0, 1 within the pair) load a tile together.
template <int ROWS, int CH>
__device__ __forceinline__ void load_tile(uint4* tile, const void* src, int64_t row_bytes,
                                          int wave, int lane) {
  constexpr int kNW = kPairThreads / cm::kWave;
  constexpr int kPer = ROWS * CH / kPairThreads;
  static_assert(kPer * kPairThreads == ROWS * CH, "tile chunks split over the pair");
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = (i * kNW + wave) * cm::kWave + lane;
    const int row = c / CH, phys = c % CH;
    const char* g = static_cast<const char*>(src) + row * row_bytes + (phys ^ swz<CH>(row)) * 16;
    cm::gemm::dma16(g, tile + (i * kNW + wave) * cm::kWave);
  }
}

// 128 bytes at src into LDS slots slot[0..7] (eight lanes of the pair's first wavefront).
__device__ __forceinline__ void load_vec128(uint4* slot, const void* src, int wave, int lane) {
  if (wave == 0 && lane < 8) cm::gemm::dma16(static_cast<const char*>(src) + lane * 16, slot);
}

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------------------
// Relayout: fp16 natural and/or transposed copies of a [heads][N][D] tensor in the padded
// position space, and optionally Delta = rowsum(X * O) (X = dO).
struct Job {
  const void* src;
  int64_t sh, st;       // element strides of src (head, token); d is contiguous
  _Float16* nat;        // [heads][n_pad][D] or null
  _Float16* tr;         // [heads][D][n_pad] (16-groups permuted) or null
  const _Float16* o;    // with delta: O, element (t, h, d) at o[t * so_t + h * D + d]
  float* delta;         // [heads][n_pad] or null
  int64_t so_t;
  int dtype;
  int heads;
  Rope rope;            // rotate the rows on the way (q and k of a fused RoPE), or cos == nullptr
};

struct Jobs {
  Job job[4];
  int first[4];  // first blockIdx.y of each job
  int n;
};

__global__ __launch_bounds__(256) void attn_relayout_kernel(Jobs jobs, const Rows* rows_p,
                                                            int n_tokens, int n_pad) {
  __shared__ _Float16 tile[kD * kBlk];  // transposed staging [d][slot]
  const Rows& rows = *rows_p;
  const Where where = locate(rows, blockIdx.x, n_tokens, n_pad);
  if (!where.live) return;
  const int y = blockIdx.y;
  // the job of this blockIdx.y, selected with static indices only
  Job job = jobs.job[0];
  int first = 0;
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    if (i < jobs.n && y >= jobs.first[i]) {
      job = jobs.job[i];
      first = jobs.first[i];
    }
  }
  const int h = y - first;
  const int b = blockIdx.x;
  const int len = where.len;
  const int local0 = (b - where.pstart / kBlk) * kBlk;
  const int pos0 = b * kBlk;
  // A thread takes chunks c = threadIdx.x + 256 i (token c / 16, 8 values of d at 8 (c % 16)).
  // All of its loads are issued before any store (the jobs' pointers carry no aliasing
  // information, so loads written after a store would wait for it): one memory round trip per
  // block instead of one per chunk. The arithmetic, and so every bit, is the per-chunk one.
  constexpr int kIt = kBlk * (kD / 8) / 256;
  static_assert(kIt * 256 == kBlk * (kD / 8), "whole chunks per thread");
  const bool rot = job.rope.cos != nullptr;
  float xv[kIt][8], cv[kIt][8], sv[kIt][8];
  half8 ov[kIt];
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int c = threadIdx.x + 256 * it;
    const int t = c / (kD / 8), ch = c % (kD / 8);
    const int local = local0 + t;
    const bool ok = local < len;
    const int64_t tok = where.start + local;
    if (ok) {
      load8f(job.src, job.dtype, h * job.sh + tok * job.st + ch * 8, xv[it]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[it][i] = 0.0f;
    }
    if (rot) {
      const int64_t ct = ok ? tok : where.start;  // pads: any row of the batch's tables
      const float* cr = job.rope.cos + ct * job.rope.cs_t + ch * 8;
      const float* sr = job.rope.sin + ct * job.rope.cs_t + ch * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        cv[it][i] = cr[i];
        sv[it][i] = sr[i];
      }
    }
    if (job.delta)
      ov[it] = ok ? *reinterpret_cast<const half8*>(job.o + tok * job.so_t + h * kD + ch * 8)
                  : zero8();
  }
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int c = threadIdx.x + 256 * it;
    const int t = c / (kD / 8), ch = c % (kD / 8);
    const bool ok = local0 + t < len;
    half8 x;
    if (!rot) {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = static_cast<_Float16>(xv[it][i]);
    } else {
      // the partner of chunk ch (d +- 64) is chunk ch ^ 8, held by the lane 8 away (a token's
      // 16 chunks are 16 consecutive lanes, every lane of the loop active)
      float pv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) pv[i] = __shfl_xor(xv[it][i], 8, cm::kWave);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        x[i] = static_cast<_Float16>(ch < 8 ? rot_minus(xv[it][i], pv[i], cv[it][i], sv[it][i])
                                            : rot_plus(xv[it][i], pv[i], cv[it][i], sv[it][i]));
    }
    if (job.nat)
      *reinterpret_cast<half8*>(job.nat + (static_cast<int64_t>(h) * n_pad + pos0 + t) * kD +
                                ch * 8) = x;
    if (job.tr) {
      // row d of the staging tile holds its 8-slot chunks XOR-swizzled by (d / 8) % 8, so the 16
      // lanes of one token (16 values of d eight apart) write to 8 distinct banks, not one
      const int slot = ((t & ~15) | perm16(t & 15)) ^ ((ch & 7) << 3);
#pragma unroll
      for (int i = 0; i < 8; ++i) tile[(ch * 8 + i) * kBlk + slot] = x[i];
    }
    if (job.delta) {
      float d = 0.0f;
      if (ok) {
#pragma unroll
        for (int i = 0; i < 8; ++i) d += static_cast<float>(x[i]) * static_cast<float>(ov[it][i]);
      }
      // the 16 chunks of a token are 16 consecutive lanes
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) d += __shfl_xor(d, m, cm::kWave);
      if (ch == 0) job.delta[static_cast<int64_t>(h) * n_pad + pos0 + t] = d;
    }
  }
  if (!job.tr) return;
  __syncthreads();
  for (int c = threadIdx.x; c < kD * (kBlk / 8); c += 256) {
    const int d = c / (kBlk / 8), ch = c % (kBlk / 8);
    const int pc = ch ^ ((d >> 3) & 7);
    *reinterpret_cast<uint4*>(job.tr + (static_cast<int64_t>(h) * kD + d) * n_pad + pos0 +
                              ch * 8) = *reinterpret_cast<const uint4*>(tile + d * kBlk + pc * 8);
  }
}

// ---------------------------------------------------------------------------------------------
// The three attention kernels run four wavefronts per block in two pairs. Both pairs own the same
// 64 queries (or keys), wavefront 2p + w the 32 of half w; the serial loop over the other side's
// blocks is split between the pairs (pair p takes every other block), each pair double-buffers
// its own tiles in its own LDS region, and at the end pair 1 hands its partial results to pair 0
// through that region. Both pairs run the same number of iterations (one barrier each).

// Forward. Block (b, h): 64 queries of one row, query head h (key/value head h / hpg). Pair p
// takes the row's 64-key blocks p, p + 2, ... up to the diagonal block qb.
constexpr int kKTile = kBlk * (kD / 8);   // K tile: 64 keys x 16 chunks
constexpr int kVTile = kD * (kBlk / 8);   // V^T tile: 128 d x 8 chunks

__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(
    const void* __restrict__ q, int q_dtype, int64_t sq_h, int64_t sq_t,
    const _Float16* __restrict__ k16, const _Float16* __restrict__ vt16,
    const Rows* __restrict__ rows_p, int n_tokens, int n_pad, int hpg, int H, float c_log2,
    _Float16* __restrict__ out, float* __restrict__ lse2, int q_padded) {
  constexpr int kStage = kKTile + kVTile;
  __shared__ uint4 lds[2][2][kStage];  // [pair][stage]
  const Rows& rows = *rows_p;
  const int h = blockIdx.x, g = h / hpg;
  const int b = heavy_first_query_block();
  const Where where = locate(rows, b, n_tokens, n_pad);
  if (!where.live) return;
  const int qb = b - where.pstart / kBlk;
  const int len = where.len;
  const int p0 = where.pstart;
  const int lane = threadIdx.x % cm::kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / cm::kWave);
  const int pair = wave >> 1, wq = wave & 1;
  const int hh = lane / 32, ln = lane % 32;
  const int ql = qb * kBlk + wq * 32 + ln;  // query position in the row
  const bool q_ok = ql < len;
  const int n_it = (qb + 2) / 2;

  const _Float16* kbase = k16 + (static_cast<int64_t>(g) * n_pad + p0) * kD;
  const _Float16* vbase = vt16 + static_cast<int64_t>(g) * kD * n_pad + p0;
  auto issue = [&](int jb, int st) {
    load_tile<kBlk, kD / 8>(lds[pair][st], kbase + jb * kBlk * kD, kD * 2, wq, lane);
    load_tile<kD, kBlk / 8>(lds[pair][st] + kKTile, vbase + jb * kBlk, n_pad * 2, wq, lane);
  };
  if (pair <= qb) issue(pair, 0);

  half8 qf[kD / 16];
  {
    // q as given (token rows), or its rotated fp16 copy in the padded positions (fused RoPE)
    const int64_t at = q_padded ? p0 + (q_ok ? ql : 0) : where.start + (q_ok ? ql : 0);
    const int64_t off = h * sq_h + at * sq_t;
#pragma unroll
    for (int ds = 0; ds < kD / 16; ++ds)
      qf[ds] = q_ok ? load8(q, q_dtype, off + ds * 16 + hh * 8) : zero8();
  }
  floatx16 o[kD / 32];
#pragma unroll
  for (int i = 0; i < kD / 32; ++i) o[i] = zero16();
  float m = -__builtin_huge_valf(), l = 0.0f;  // reference max (log2 domain) and sum

  for (int it = 0; it < n_it; ++it) {
    const int jb = 2 * it + pair, st = it & 1;
    cm::gemm::wait_vmcnt<0>();
    cm::gemm::lds_barrier();
    if (jb + 2 <= qb) issue(jb + 2, st ^ 1);
    if (jb > qb) continue;  // pair 1's last iteration when qb is even
    const uint4* kt = lds[pair][st];
    const uint4* vt = kt + kKTile;
    floatx16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = zero16();
#pragma unroll
      for (int ds = 0; ds < kD / 16; ++ds)
        s[t] = mfma(frag<kD / 8>(kt, t * 32 + ln, ds * 2 + hh), qf[ds], s[t]);
    }
    if (jb == qb) {  // the diagonal block: keys after the query are masked
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = jb * kBlk + t * 32 + (e / 4) * 8 + hh * 4 + e % 4;
          s[t][e] = key <= ql ? s[t][e] : -__builtin_huge_valf();
        }
    }
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[t][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, cm::kWave));
    // The exponentials are taken against a reference max m that moves only when some row's max
    // exceeds it by more than 2^8 (then every row of the wavefront moves to its own max and O
    // and l are rescaled): probabilities stay <= 256, exact to fp16's relative precision, and
    // most blocks skip the rescale.
    float alpha = 1.0f;
    if (__builtin_amdgcn_ballot_w64(mx * c_log2 > m + 8.0f)) {
      const float m_new = fmaxf(m, mx * c_log2);
      alpha = exp2_raw(m - m_new);
      m = m_new;
#pragma unroll
      for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
    }
    const float m_new = m;
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = exp2_raw(__builtin_fmaf(s[t][e], c_log2, -m_new));
        s[t][e] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 32, cm::kWave);
    l = l * alpha + sum;
    half8 pf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pf[ks] = frag_of(s[ks / 2], ks % 2);
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        o[dt] = mfma(frag<kBlk / 8>(vt, dt * 32 + ln, ks * 2 + hh), pf[ks], o[dt]);
  }

  // pair 1 hands (o, m, l) of its blocks to pair 0 through its LDS region
  cm::gemm::lds_barrier();
  float* xf = reinterpret_cast<float*>(lds[1][0]) + wq * 66 * cm::kWave + lane;
  if (pair == 1) {
#pragma unroll
    for (int i = 0; i < kD / 2; ++i) xf[i * cm::kWave] = o[i / 16][i % 16];
    xf[64 * cm::kWave] = m;
    xf[65 * cm::kWave] = l;
  }
  cm::gemm::lds_barrier();
  if (pair == 1) return;
  const float m1 = xf[64 * cm::kWave], l1 = xf[65 * cm::kWave];
  const float mt = fmaxf(m, m1);
  const float a0 = exp2_raw(m - mt), a1 = exp2_raw(m1 - mt);  // a1 = 0 when pair 1 had none
  l = l * a0 + l1 * a1;
  if (hh == 0) lse2[static_cast<int64_t>(h) * n_pad + p0 + ql] = mt + __log2f(l);
  if (!q_ok) return;
  const float inv = 1.0f / l;
  _Float16* orow = out + (static_cast<int64_t>(where.start + ql) * H + h) * kD;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      h4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = g4 * 4 + i;
        v[i] = static_cast<_Float16>((o[dt][e] * a0 + xf[(dt * 16 + e) * cm::kWave] * a1) * inv);
      }
      *reinterpret_cast<h4*>(orow + dt * 32 + g4 * 8 + hh * 4) = v;
    }
}

// ---------------------------------------------------------------------------------------------
// Backward, dK and dV. Block (b, h): 64 keys of one row against query head h; pair p takes the
// row's 32-query tiles qt_first + p, qt_first + p + 2, ... from the block's first key on. Writes
// the head's partial dK (times the softmax scale) and dV, fp32 [H][n_pad][D]. Queries past the
// row end need no mask: their q and dO rows are zero, so they add exactly zero.
constexpr int kQTile = 32 * (kD / 8);   // Q / dO tile: 32 queries x 16 chunks
constexpr int kQTTile = kD * (32 / 8);  // Q^T / dO^T tile: 128 d x 4 chunks
constexpr int kDkdvVec = 2 * kQTile + 2 * kQTTile;  // lse (8 chunks) and Delta (8) follow
constexpr int kDkdvStage = kDkdvVec + 16;

// The operands of the backward's dK/dV and dQ blocks (one launch runs both).
struct BwdArgs {
  const _Float16* q16;
  const _Float16* qt16;
  const _Float16* do16;
  const _Float16* dot16;
  const _Float16* k16;
  const _Float16* v16;
  const _Float16* kt16;
  const float* lse2;
  const float* delta;
  const Rows* rows;
  int n_tokens, n_pad, hpg, H;
  float c_log2, scale;
  float* dk_part;
  float* dv_part;
  void* dq;         // fp32 or fp16, [H][N][D] or [N][H][D] with tok_major
  int tok_major;
  float* dq_rot;    // fused RoPE: dQ of the rotated q, [H][n_pad][D] fp32, or null
};

// raw: the workgroup's LDS, 4 stages of kDkdvStage
__device__ __forceinline__ void bwd_dkdv_block(const BwdArgs& a, int h, int b, uint4* raw) {
  constexpr int kVec = kDkdvVec;
  constexpr int kStage = kDkdvStage;
  auto lds = reinterpret_cast<uint4 (*)[2][kStage]>(raw);  // [pair][stage]
  const _Float16* __restrict__ q16 = a.q16;
  const _Float16* __restrict__ qt16 = a.qt16;
  const _Float16* __restrict__ do16 = a.do16;
  const _Float16* __restrict__ dot16 = a.dot16;
  const _Float16* __restrict__ k16 = a.k16;
  const _Float16* __restrict__ v16 = a.v16;
  const float* __restrict__ lse2 = a.lse2;
  const float* __restrict__ delta = a.delta;
  const int n_pad = a.n_pad;
  const float c_log2 = a.c_log2, scale = a.scale;
  const Rows& rows = *a.rows;
  const int g = h / a.hpg;
  const Where where = locate(rows, b, a.n_tokens, n_pad);
  if (!where.live) return;
  const int kb = b - where.pstart / kBlk;
  const int len = where.len;
  const int p0 = where.pstart;
  const int lane = threadIdx.x % cm::kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / cm::kWave);
  const int pair = wave >> 1, wq = wave & 1;
  const int hh = lane / 32, ln = lane % 32;
  const int key0 = kb * kBlk + wq * 32;  // first key of the wavefront
  const int key = key0 + ln;

  const int64_t hq = static_cast<int64_t>(h) * n_pad;
  auto issue = [&](int qt, int st) {
    const int64_t pos = p0 + qt * 32;
    uint4* t = lds[pair][st];
    load_tile<32, kD / 8>(t, q16 + (hq + pos) * kD, kD * 2, wq, lane);
    load_tile<32, kD / 8>(t + kQTile, do16 + (hq + pos) * kD, kD * 2, wq, lane);
    load_tile<kD, 32 / 8>(t + 2 * kQTile, qt16 + static_cast<int64_t>(h) * kD * n_pad + pos,
                          n_pad * 2, wq, lane);
    load_tile<kD, 32 / 8>(t + 2 * kQTile + kQTTile,
                          dot16 + static_cast<int64_t>(h) * kD * n_pad + pos, n_pad * 2, wq,
                          lane);
    load_vec128(t + kVec, lse2 + hq + pos, wq, lane);
    load_vec128(t + kVec + 8, delta + hq + pos, wq, lane);
  };
  const int qt_first = 2 * kb;
  const int qt_end = (len + 31) / 32;
  const int n_it = (qt_end - qt_first + 1) / 2;
  if (qt_first + pair < qt_end) issue(qt_first + pair, 0);

  half8 kf[kD / 16], vf[kD / 16];
  {
    const int64_t off = (static_cast<int64_t>(g) * n_pad + p0 + key) * kD;
#pragma unroll
    for (int ds = 0; ds < kD / 16; ++ds) {
      kf[ds] = *reinterpret_cast<const half8*>(k16 + off + ds * 16 + hh * 8);
      vf[ds] = *reinterpret_cast<const half8*>(v16 + off + ds * 16 + hh * 8);
    }
  }
  floatx16 dk[kD / 32], dv[kD / 32];
#pragma unroll
  for (int i = 0; i < kD / 32; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  for (int it = 0; it < n_it; ++it) {
    const int qt = qt_first + 2 * it + pair, st = it & 1;
    cm::gemm::wait_vmcnt<0>();
    cm::gemm::lds_barrier();
    if (qt + 2 < qt_end) issue(qt + 2, st ^ 1);
    if (qt >= qt_end) continue;           // pair 1's last iteration
    if (qt * 32 + 31 < key0) continue;    // the tile's queries all precede this wavefront's keys
    const uint4* qs = lds[pair][st];
    const uint4* dos = qs + kQTile;
    const uint4* qts = qs + 2 * kQTile;
    const uint4* dots = qts + kQTTile;
    // lse and Delta of the lane's 16 queries qt*32 + (e/4)*8 + hh*4 + e%4
    const float4* lv = reinterpret_cast<const float4*>(qs + kVec);
    const float4* dlv = reinterpret_cast<const float4*>(qs + kVec + 8);
    floatx16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ds = 0; ds < kD / 16; ++ds) {
      s = mfma(frag<kD / 8>(qs, ln, ds * 2 + hh), kf[ds], s);
      dp = mfma(frag<kD / 8>(dos, ln, ds * 2 + hh), vf[ds], dp);
    }
    const bool diag = qt * 32 < key0 + 31;  // some query of the tile precedes some key
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const float4 lq = lv[g4 * 2 + hh], dq4 = dlv[g4 * 2 + hh];
      const float lsv[4] = {lq.x, lq.y, lq.z, lq.w}, dlq[4] = {dq4.x, dq4.y, dq4.z, dq4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = g4 * 4 + i;
        float p = exp2_raw(__builtin_fmaf(s[e], c_log2, -lsv[i]));
        if (diag) p = key <= qt * 32 + g4 * 8 + hh * 4 + i ? p : 0.0f;
        s[e] = p;
        dp[e] = p * (dp[e] - dlq[i]);
      }
    }
    half8 pf[2], sf[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      pf[j] = frag_of(s, j);
      sf[j] = frag_of(dp, j);
    }
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        dv[dt] = mfma(frag<32 / 8>(dots, dt * 32 + ln, j * 2 + hh), pf[j], dv[dt]);
        dk[dt] = mfma(frag<32 / 8>(qts, dt * 32 + ln, j * 2 + hh), sf[j], dk[dt]);
      }
  }

  cm::gemm::lds_barrier();
  float* xf = reinterpret_cast<float*>(lds[1][0]) + wq * 128 * cm::kWave + lane;
  if (pair == 1) {
#pragma unroll
    for (int i = 0; i < kD / 2; ++i) {
      xf[i * cm::kWave] = dk[i / 16][i % 16];
      xf[(64 + i) * cm::kWave] = dv[i / 16][i % 16];
    }
  }
  cm::gemm::lds_barrier();
  if (pair == 1) return;
  float* dkr = a.dk_part + (hq + p0 + key) * kD;
  float* dvr = a.dv_part + (hq + p0 + key) * kD;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = dt * 32 + g4 * 8 + hh * 4, e = dt * 16 + g4 * 4;
      float4 a, c;
      a.x = (dk[dt][g4 * 4] + xf[e * cm::kWave]) * scale;
      a.y = (dk[dt][g4 * 4 + 1] + xf[(e + 1) * cm::kWave]) * scale;
      a.z = (dk[dt][g4 * 4 + 2] + xf[(e + 2) * cm::kWave]) * scale;
      a.w = (dk[dt][g4 * 4 + 3] + xf[(e + 3) * cm::kWave]) * scale;
      c.x = dv[dt][g4 * 4] + xf[(64 + e) * cm::kWave];
      c.y = dv[dt][g4 * 4 + 1] + xf[(65 + e) * cm::kWave];
      c.z = dv[dt][g4 * 4 + 2] + xf[(66 + e) * cm::kWave];
      c.w = dv[dt][g4 * 4 + 3] + xf[(67 + e) * cm::kWave];
      *reinterpret_cast<float4*>(dkr + d) = a;
      *reinterpret_cast<float4*>(dvr + d) = c;
    }
}

// ---------------------------------------------------------------------------------------------
// Backward, dQ. Block (b, h): 64 queries of one row, head h; pair p takes the 32-key tiles p,
// p + 2, ... up to the diagonal.
constexpr int kKVTile = 32 * (kD / 8);  // K / V tile: 32 keys x 16 chunks
constexpr int kKTTile = kD * (32 / 8);  // K^T tile: 128 d x 4 chunks

constexpr int kDqStage = 2 * kKVTile + kKTTile;

template <typename OT>
__device__ __forceinline__ void bwd_dq_block(const BwdArgs& a, int h, int b, uint4* raw) {
  constexpr int kStage = kDqStage;
  auto lds = reinterpret_cast<uint4 (*)[2][kStage]>(raw);  // [pair][stage]
  const _Float16* __restrict__ q16 = a.q16;
  const _Float16* __restrict__ do16 = a.do16;
  const _Float16* __restrict__ k16 = a.k16;
  const _Float16* __restrict__ v16 = a.v16;
  const _Float16* __restrict__ kt16 = a.kt16;
  const float* __restrict__ lse2 = a.lse2;
  const float* __restrict__ delta = a.delta;
  const int n_tokens = a.n_tokens, n_pad = a.n_pad, tok_major = a.tok_major;
  const float c_log2 = a.c_log2, scale = a.scale;
  float* __restrict__ dq_rot = a.dq_rot;
  OT* __restrict__ dq = static_cast<OT*>(a.dq);
  const Rows& rows = *a.rows;
  const int g = h / a.hpg;
  const Where where = locate(rows, b, n_tokens, n_pad);
  if (!where.live) return;
  const int qb = b - where.pstart / kBlk;
  const int len = where.len;
  const int p0 = where.pstart;
  const int lane = threadIdx.x % cm::kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / cm::kWave);
  const int pair = wave >> 1, wq = wave & 1;
  const int hh = lane / 32, ln = lane % 32;
  const int q0 = qb * kBlk + wq * 32;  // first query of the wavefront
  const int ql = q0 + ln;

  const int64_t gk = static_cast<int64_t>(g) * n_pad;
  auto issue = [&](int kt, int st) {
    const int64_t pos = p0 + kt * 32;
    uint4* t = lds[pair][st];
    load_tile<32, kD / 8>(t, k16 + (gk + pos) * kD, kD * 2, wq, lane);
    load_tile<32, kD / 8>(t + kKVTile, v16 + (gk + pos) * kD, kD * 2, wq, lane);
    load_tile<kD, 32 / 8>(t + 2 * kKVTile, kt16 + static_cast<int64_t>(g) * kD * n_pad + pos,
                          n_pad * 2, wq, lane);
  };
  const int n_it = qb + 1;  // 32-key tiles 0 .. 2 qb + 1, every other one per pair
  issue(pair, 0);

  const int64_t at = static_cast<int64_t>(h) * n_pad + p0 + ql;
  half8 qf[kD / 16], of[kD / 16];
#pragma unroll
  for (int ds = 0; ds < kD / 16; ++ds) {
    qf[ds] = *reinterpret_cast<const half8*>(q16 + at * kD + ds * 16 + hh * 8);
    of[ds] = *reinterpret_cast<const half8*>(do16 + at * kD + ds * 16 + hh * 8);
  }
  const float ls = lse2[at], dl = delta[at];
  floatx16 acc[kD / 32];
#pragma unroll
  for (int i = 0; i < kD / 32; ++i) acc[i] = zero16();

  for (int it = 0; it < n_it; ++it) {
    const int kt = 2 * it + pair, st = it & 1;
    cm::gemm::wait_vmcnt<0>();
    cm::gemm::lds_barrier();
    if (kt + 2 < 2 * n_it) issue(kt + 2, st ^ 1);
    if (kt * 32 > q0 + 31) continue;  // the tile's keys all follow this wavefront's queries
    const uint4* ks = lds[pair][st];
    const uint4* vs = ks + kKVTile;
    const uint4* kts = ks + 2 * kKVTile;
    floatx16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ds = 0; ds < kD / 16; ++ds) {
      s = mfma(frag<kD / 8>(ks, ln, ds * 2 + hh), qf[ds], s);
      dp = mfma(frag<kD / 8>(vs, ln, ds * 2 + hh), of[ds], dp);
    }
    const bool diag = kt * 32 + 31 > q0;  // some key of the tile follows some query
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float p = exp2_raw(__builtin_fmaf(s[e], c_log2, -ls));
      if (diag) p = kt * 32 + (e / 4) * 8 + hh * 4 + e % 4 <= ql ? p : 0.0f;
      dp[e] = p * (dp[e] - dl);
    }
    half8 sf[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) sf[j] = frag_of(dp, j);
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[dt] = mfma(frag<32 / 8>(kts, dt * 32 + ln, j * 2 + hh), sf[j], acc[dt]);
  }

  cm::gemm::lds_barrier();
  float* xf = reinterpret_cast<float*>(lds[1][0]) + wq * 64 * cm::kWave + lane;
  if (pair == 1) {
#pragma unroll
    for (int i = 0; i < kD / 2; ++i) xf[i * cm::kWave] = acc[i / 16][i % 16];
  }
  cm::gemm::lds_barrier();
  if (pair == 1 || ql >= len) return;
  // dq is [H][N][D], or [N][H][D] with tok_major
  const int64_t tok = where.start + ql;
  if (dq_rot != nullptr) {
    // fused RoPE: the gradient of the rotated q, [H][n_pad][D] fp32, which the reduce launch
    // takes back through the transposed rotation (reading the cos / sin rows coalesced there)
    float* rrow = dq_rot + (static_cast<int64_t>(h) * n_pad + p0 + ql) * kD;
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        rrow[dt * 32 + (e / 4) * 8 + hh * 4 + e % 4] =
            (acc[dt][e] + xf[(dt * 16 + e) * cm::kWave]) * scale;
    return;
  }
  OT* row = dq + (tok_major ? tok * a.H + h : static_cast<int64_t>(h) * n_tokens + tok) * kD;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      row[dt * 32 + (e / 4) * 8 + hh * 4 + e % 4] =
          cm::from_f32<OT>((acc[dt][e] + xf[(dt * 16 + e) * cm::kWave]) * scale);
}

// dK, dV = sum of the partials of the query heads of each group, [G][N][D] (or [N][G][D]) in the
// output dtype.
// ---------------------------------------------------------------------------------------------
// The backward's dK/dV and dQ blocks in one launch: blockIdx.x < H is the dK/dV block
// (blockIdx.y, head blockIdx.x), the rest the dQ block (gridDim.y - 1 - blockIdx.y, head
// blockIdx.x - H). The two sets are independent (different outputs, the same relayout inputs),
// and each has a few heavy blocks (a long row's first key blocks, its last query blocks) among
// many light ones: dispatched together, heaviest first in both, the light blocks of one fill the
// CUs the other's heavy blocks leave idle. The LDS holds the larger of the two stage rings.
constexpr int kBwdLds = 4 * (kDkdvStage > kDqStage ? kDkdvStage : kDqStage);

template <typename OT>
__global__ __launch_bounds__(kThreads) void attn_bwd_kernel(BwdArgs a) {
  __shared__ uint4 raw[kBwdLds];
  const int x = blockIdx.x;
  if (x < a.H) {
    bwd_dkdv_block(a, x, blockIdx.y, raw);  // a row's first key blocks (the most queries) first
  } else {
    bwd_dq_block<OT>(a, x - a.H, static_cast<int>(gridDim.y) - 1 - blockIdx.y, raw);
  }
}

// ---------------------------------------------------------------------------------------------
// Thread (position, 4 values of d) of key/value head blockIdx.y. With a fused RoPE, dK is the
// gradient of the rotated k taken back through the transposed rotation (the partner values,
// d +- 64, are 16 lanes away: a position's 32 threads are consecutive lanes and return together),
// and blockIdx.y = G + h takes query head h's gradient (dq_rot, written by the dQ kernel) back
// the same way into dq.
struct DqRope {
  const float* rot;  // [H][n_pad][D]
  void* dq;          // [N][H][D] (token-major) or [H][N][D]
  int f32;           // dq's dtype: fp32, else fp16
  int H;
};

__device__ __forceinline__ float4 rotate_back(float4 v, int d, const Rope& rope, int64_t tok) {
  const float4 p = make_float4(__shfl_xor(v.x, 16, cm::kWave), __shfl_xor(v.y, 16, cm::kWave),
                               __shfl_xor(v.z, 16, cm::kWave), __shfl_xor(v.w, 16, cm::kWave));
  const float* cr = rope.cos + tok * rope.cs_t + d;
  const float* sp = rope.sin + tok * rope.cs_t + (d < 64 ? d + 64 : d - 64);  // the partner's
  if (d < 64)
    return make_float4(rot_plus(v.x, p.x, cr[0], sp[0]), rot_plus(v.y, p.y, cr[1], sp[1]),
                       rot_plus(v.z, p.z, cr[2], sp[2]), rot_plus(v.w, p.w, cr[3], sp[3]));
  return make_float4(rot_minus(v.x, p.x, cr[0], sp[0]), rot_minus(v.y, p.y, cr[1], sp[1]),
                     rot_minus(v.z, p.z, cr[2], sp[2]), rot_minus(v.w, p.w, cr[3], sp[3]));
}

template <typename T>
__device__ __forceinline__ void store4(T* p, float4 v) {
  p[0] = cm::from_f32<T>(v.x); p[1] = cm::from_f32<T>(v.y);
  p[2] = cm::from_f32<T>(v.z); p[3] = cm::from_f32<T>(v.w);
}

template <typename KT, typename VT>
__global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(
    const float* __restrict__ dk_part, const float* __restrict__ dv_part,
    const Rows* __restrict__ rows_p, int n_tokens, int n_pad, int hpg, KT* __restrict__ dk,
    VT* __restrict__ dv, int tok_major, Rope rope, DqRope dqr) {
  const Rows& rows = *rows_p;
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int pos = i / (kD / 4), d = (i % (kD / 4)) * 4;
  // a workgroup's 8 positions share one 64-position block (blockIdx.x * 8 .. + 7)
  const Where where = locate(rows, __builtin_amdgcn_readfirstlane(pos / kBlk), n_tokens, n_pad);
  if (pos >= n_pad || !where.live) return;
  const int local = pos - where.pstart;
  if (local >= where.len) return;
  const int64_t tok = where.start + local;
  const int G = static_cast<int>(gridDim.y) - (dqr.rot != nullptr ? dqr.H : 0);
  if (static_cast<int>(blockIdx.y) >= G) {  // query head blockIdx.y - G of a fused RoPE
    const int h = blockIdx.y - G;
    const float4 gq = *reinterpret_cast<const float4*>(
        dqr.rot + (static_cast<int64_t>(h) * n_pad + pos) * kD + d);
    const float4 o = rotate_back(gq, d, rope, tok);
    const int64_t at = (tok_major ? tok * dqr.H + h : static_cast<int64_t>(h) * n_tokens + tok) * kD + d;
    if (dqr.f32)
      store4(static_cast<float*>(dqr.dq) + at, o);
    else
      store4(static_cast<_Float16*>(dqr.dq) + at, o);
    return;
  }
  const int g = blockIdx.y;
  float4 sk = make_float4(0.f, 0.f, 0.f, 0.f), sv = sk;
  for (int j = 0; j < hpg; ++j) {
    const int64_t at = ((static_cast<int64_t>(g) * hpg + j) * n_pad + pos) * kD + d;
    const float4 a = *reinterpret_cast<const float4*>(dk_part + at);
    const float4 c = *reinterpret_cast<const float4*>(dv_part + at);
    sk.x += a.x; sk.y += a.y; sk.z += a.z; sk.w += a.w;
    sv.x += c.x; sv.y += c.y; sv.z += c.z; sv.w += c.w;
  }
  // dK, dV are [G][N][D], or [N][G][D] with tok_major
  const int64_t o = (tok_major ? tok * G + g : static_cast<int64_t>(g) * n_tokens + tok) * kD + d;
  if (rope.cos != nullptr) sk = rotate_back(sk, d, rope, tok);
  store4(dk + o, sk);
  store4(dv + o, sv);
}

// ---------------------------------------------------------------------------------------------
// Host side.
int build_rows(const int64_t* bounds, int n_rows, Rows& rows, int64_t& n_pad) {
  if (!bounds || n_rows < 1 || n_rows > kMaxRows || bounds[0] != 0) return hipErrorInvalidValue;
  rows.n = n_rows;
  int64_t p = 0;
  for (int r = 0; r <= n_rows; ++r) {
    if (r > 0 && bounds[r] < bounds[r - 1]) return hipErrorInvalidValue;
    if (bounds[r] > 0x3fffffff) return hipErrorInvalidValue;
    rows.start[r] = static_cast<int>(bounds[r]);
    rows.pstart[r] = static_cast<int>(p);
    if (r < n_rows) p += (bounds[r + 1] - bounds[r] + kBlk - 1) / kBlk * kBlk;
  }
  n_pad = p;
  return 0;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// 16-byte aligned base and strides that keep every 8-element chunk 16-byte aligned.
bool aligned_operand(const void* p, int dtype, int64_t sh, int64_t st) {
  const int64_t mult = dtype == CM_F32 ? 4 : 8;
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && sh % mult == 0 && st % mult == 0;
}

struct Workspace {
  char* p;
  size_t used = 0, size;
  template <typename T>
  T* take(size_t count) {
    T* at = reinterpret_cast<T*>(p + used);
    used += align256(count * sizeof(T));
    return at;
  }
};

// k16 and vt16, and q16 (the rotated q of a fused RoPE)
size_t fwd_ws_bytes(int64_t n_pad, int H, int G) {
  return 2 * align256(static_cast<size_t>(G) * n_pad * kD * 2) +
         align256(static_cast<size_t>(H) * n_pad * kD * 2);
}

// q16, do16, qt16, dot16; k16, v16, kt16; Delta; dK / dV partials and the fused RoPE's dQ
size_t bwd_ws_bytes(int64_t n_pad, int H, int G) {
  const size_t hq = align256(static_cast<size_t>(H) * n_pad * kD * 2);
  const size_t gk = align256(static_cast<size_t>(G) * n_pad * kD * 2);
  const size_t part = align256(static_cast<size_t>(H) * n_pad * kD * 4);
  return 4 * hq + 3 * gk + align256(static_cast<size_t>(H) * n_pad * 4) + 3 * part;
}

}  // namespace

extern "C" int64_t cm_attn_padded_tokens(const int64_t* bounds, int n_rows) {
  Rows rows;
  int64_t n_pad;
  if (build_rows(bounds, n_rows, rows, n_pad)) return -1;
  return n_pad;
}

extern "C" int64_t cm_attn_rows_bytes(void) { return static_cast<int64_t>(sizeof(Rows)); }

extern "C" int64_t cm_attn_rows_image(const int64_t* bounds, int n_rows, void* image) {
  Rows rows;
  int64_t n_pad;
  if (!image || build_rows(bounds, n_rows, rows, n_pad)) return -1;
  memcpy(image, &rows, sizeof(Rows));
  return n_pad;
}

extern "C" int64_t cm_attn_workspace_bytes(int64_t n_pad, int H, int G, int head_dim,
                                           int backward) {
  if (n_pad < 0 || H <= 0 || G <= 0 || head_dim != kD) return -1;
  return static_cast<int64_t>(backward ? bwd_ws_bytes(n_pad, H, G) : fwd_ws_bytes(n_pad, H, G));
}

// Launch arguments shared by both directions: the rows image (device memory, 16-byte aligned), the
// token count and a padded capacity that is a positive multiple of the block.
bool rows_args_ok(const void* rows, int64_t n_tokens, int64_t n_pad) {
  // the padded blocks are the grids' second dimension (at most 65535)
  return rows && (reinterpret_cast<uintptr_t>(rows) & 15) == 0 && n_tokens >= 0 &&
         n_tokens <= 0x3fffffff && n_pad > 0 && n_pad % kBlk == 0 && n_pad / kBlk <= 65535;
}

namespace {

// A fused RoPE's tables: none (cos == nullptr), or fp32 rows of 16-byte aligned cos / sin with a
// row stride that keeps them aligned.
bool rope_ok(const Rope& r) {
  if (r.cos == nullptr) return r.sin == nullptr;
  return r.sin != nullptr && (reinterpret_cast<uintptr_t>(r.cos) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(r.sin) & 15) == 0 && r.cs_t >= kD && r.cs_t % 4 == 0;
}

int fwd_impl(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k, int k_dtype,
             int64_t sk_h, int64_t sk_t, const void* v, int v_dtype, int64_t sv_h, int64_t sv_t,
             Rope rope, const void* rows_image, int64_t n_tokens, int64_t n_pad, int H, int G,
             int head_dim, float scale, void* out, float* lse2, void* workspace,
             int64_t workspace_bytes, void* stream) {
  CM_CHECK_ARG(head_dim == kD && H > 0 && G > 0 && H % G == 0 && H <= 65535);
  CM_CHECK_ARG((q_dtype == CM_F32 || q_dtype == CM_F16) && (k_dtype == CM_F32 || k_dtype == CM_F16) &&
               (v_dtype == CM_F32 || v_dtype == CM_F16));
  CM_CHECK_ARG(rope_ok(rope));
  if (n_tokens == 0) return 0;
  CM_CHECK_ARG(rows_args_ok(rows_image, n_tokens, n_pad));
  CM_CHECK_ARG(q && k && v && out && lse2 && workspace);
  CM_CHECK_ARG(aligned_operand(q, q_dtype, sq_h, sq_t) && aligned_operand(k, k_dtype, sk_h, sk_t) &&
               aligned_operand(v, v_dtype, sv_h, sv_t));
  CM_CHECK_ARG((reinterpret_cast<uintptr_t>(out) & 7) == 0 &&
               (reinterpret_cast<uintptr_t>(workspace) & 255) == 0);
  CM_CHECK_ARG(workspace_bytes >= static_cast<int64_t>(fwd_ws_bytes(n_pad, H, G)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace ws{static_cast<char*>(workspace), 0, static_cast<size_t>(workspace_bytes)};
  _Float16* k16 = ws.take<_Float16>(static_cast<size_t>(G) * n_pad * kD);
  _Float16* vt16 = ws.take<_Float16>(static_cast<size_t>(G) * n_pad * kD);
  _Float16* q16 = ws.take<_Float16>(static_cast<size_t>(H) * n_pad * kD);
  const Rope none{nullptr, nullptr, 0};
  const bool fused = rope.cos != nullptr;
  // with a fused RoPE, q and k are rotated on their way into the fp16 copies, and the query
  // kernel reads q's copy (in the padded positions) in place of q
  Jobs jobs{};
  jobs.job[0] = Job{k, sk_h, sk_t, k16, nullptr, nullptr, nullptr, 0, k_dtype, G, rope};
  jobs.job[1] = Job{v, sv_h, sv_t, nullptr, vt16, nullptr, nullptr, 0, v_dtype, G, none};
  jobs.job[2] = Job{q, sq_h, sq_t, q16, nullptr, nullptr, nullptr, 0, q_dtype, H, rope};
  jobs.first[1] = G;
  jobs.first[2] = 2 * G;
  jobs.n = fused ? 3 : 2;
  const int n_blocks = static_cast<int>(n_pad / kBlk);
  const Rows* rows = static_cast<const Rows*>(rows_image);
  const int nt = static_cast<int>(n_tokens), np = static_cast<int>(n_pad);
  hipLaunchKernelGGL(attn_relayout_kernel, dim3(n_blocks, 2 * G + (fused ? H : 0)), dim3(256), 0,
                     s, jobs, rows, nt, np);
  if (int st = cm::launch_status()) return st;
  const void* qa = fused ? static_cast<const void*>(q16) : q;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(H, n_blocks), dim3(kThreads), 0, s, qa,
                     fused ? CM_F16 : q_dtype, fused ? static_cast<int64_t>(n_pad) * kD : sq_h,
                     fused ? static_cast<int64_t>(kD) : sq_t, k16, vt16, rows, nt, np, H / G, H,
                     scale * 1.4426950408889634f, static_cast<_Float16*>(out), lse2,
                     fused ? 1 : 0);
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_attn_fwd(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k,
                           int k_dtype, int64_t sk_h, int64_t sk_t, const void* v, int v_dtype,
                           int64_t sv_h, int64_t sv_t, const void* rows_image, int64_t n_tokens,
                           int64_t n_pad, int H, int G, int head_dim, float scale, void* out,
                           float* lse2, void* workspace, int64_t workspace_bytes, void* stream) {
  return fwd_impl(q, q_dtype, sq_h, sq_t, k, k_dtype, sk_h, sk_t, v, v_dtype, sv_h, sv_t,
                  Rope{nullptr, nullptr, 0}, rows_image, n_tokens, n_pad, H, G, head_dim, scale,
                  out, lse2, workspace, workspace_bytes, stream);
}

extern "C" int cm_attn_fwd_rope(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t,
                                const void* k, int k_dtype, int64_t sk_h, int64_t sk_t,
                                const void* v, int v_dtype, int64_t sv_h, int64_t sv_t,
                                const float* cos, const float* sin, int64_t cs_t,
                                const void* rows_image, int64_t n_tokens, int64_t n_pad, int H,
                                int G, int head_dim, float scale, void* out, float* lse2,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  CM_CHECK_ARG(cos != nullptr);
  return fwd_impl(q, q_dtype, sq_h, sq_t, k, k_dtype, sk_h, sk_t, v, v_dtype, sv_h, sv_t,
                  Rope{cos, sin, cs_t}, rows_image, n_tokens, n_pad, H, G, head_dim, scale, out,
                  lse2, workspace, workspace_bytes, stream);
}

namespace {

int bwd_impl(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k, int k_dtype,
             int64_t sk_h, int64_t sk_t, const void* v, int v_dtype, int64_t sv_h, int64_t sv_t,
             Rope rope, const void* out, const void* dout, const float* lse2,
             const void* rows_image, int64_t n_tokens, int64_t n_pad, int H, int G, int head_dim,
             float scale, void* dq, int dq_dtype, void* dk, int dk_dtype, void* dv, int dv_dtype,
             int grads_token_major, void* workspace, int64_t workspace_bytes, void* stream) {
  // the backward's grid holds 2 H workgroups along x
  CM_CHECK_ARG(head_dim == kD && H > 0 && G > 0 && H % G == 0 && H <= 32767);
  CM_CHECK_ARG((q_dtype == CM_F32 || q_dtype == CM_F16) && (k_dtype == CM_F32 || k_dtype == CM_F16) &&
               (v_dtype == CM_F32 || v_dtype == CM_F16));
  CM_CHECK_ARG((dq_dtype == CM_F32 || dq_dtype == CM_F16) &&
               (dk_dtype == CM_F32 || dk_dtype == CM_F16) &&
               (dv_dtype == CM_F32 || dv_dtype == CM_F16));
  CM_CHECK_ARG(rope_ok(rope));
  if (n_tokens == 0) return 0;
  CM_CHECK_ARG(rows_args_ok(rows_image, n_tokens, n_pad));
  CM_CHECK_ARG(q && k && v && out && dout && lse2 && dq && dk && dv && workspace);
  CM_CHECK_ARG(aligned_operand(q, q_dtype, sq_h, sq_t) && aligned_operand(k, k_dtype, sk_h, sk_t) &&
               aligned_operand(v, v_dtype, sv_h, sv_t));
  CM_CHECK_ARG((reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
               (reinterpret_cast<uintptr_t>(dout) & 15) == 0 &&
               (reinterpret_cast<uintptr_t>(lse2) & 15) == 0 &&
               (reinterpret_cast<uintptr_t>(workspace) & 255) == 0);
  CM_CHECK_ARG(workspace_bytes >= static_cast<int64_t>(bwd_ws_bytes(n_pad, H, G)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace ws{static_cast<char*>(workspace), 0, static_cast<size_t>(workspace_bytes)};
  const size_t nq = static_cast<size_t>(H) * n_pad * kD, nk = static_cast<size_t>(G) * n_pad * kD;
  _Float16* q16 = ws.take<_Float16>(nq);
  _Float16* do16 = ws.take<_Float16>(nq);
  _Float16* qt16 = ws.take<_Float16>(nq);
  _Float16* dot16 = ws.take<_Float16>(nq);
  _Float16* k16 = ws.take<_Float16>(nk);
  _Float16* v16 = ws.take<_Float16>(nk);
  _Float16* kt16 = ws.take<_Float16>(nk);
  float* delta = ws.take<float>(static_cast<size_t>(H) * n_pad);
  float* dk_part = ws.take<float>(nq);
  float* dv_part = ws.take<float>(nq);
  // with a fused RoPE, dQ of the rotated q ([H][n_pad][D] fp32) for the head-sum launch to rotate
  float* dq_rot_ws = ws.take<float>(nq);
  float* dq_rot = rope.cos != nullptr ? dq_rot_ws : nullptr;
  const int np = static_cast<int>(n_pad), nt = static_cast<int>(n_tokens);
  const int n_blocks = np / kBlk;
  const Rows* rows = static_cast<const Rows*>(rows_image);
  const Rope none{nullptr, nullptr, 0};
  // dO and O: [N][H][D] contiguous (the forward's output layout); q and k rotated again on the
  // way when the RoPE is fused
  Jobs jobs{};
  jobs.job[0] = Job{q, sq_h, sq_t, q16, qt16, nullptr, nullptr, 0, q_dtype, H, rope};
  jobs.job[1] = Job{dout, kD, static_cast<int64_t>(H) * kD, do16, dot16,
                    static_cast<const _Float16*>(out), delta, static_cast<int64_t>(H) * kD,
                    CM_F16, H, none};
  jobs.job[2] = Job{k, sk_h, sk_t, k16, kt16, nullptr, nullptr, 0, k_dtype, G, rope};
  jobs.job[3] = Job{v, sv_h, sv_t, v16, nullptr, nullptr, nullptr, 0, v_dtype, G, none};
  jobs.first[1] = H;
  jobs.first[2] = 2 * H;
  jobs.first[3] = 2 * H + G;
  jobs.n = 4;
  hipLaunchKernelGGL(attn_relayout_kernel, dim3(n_blocks, 2 * H + 2 * G), dim3(256), 0, s, jobs,
                     rows, nt, np);
  if (int st = cm::launch_status()) return st;
  const int tm = grads_token_major ? 1 : 0;
  const BwdArgs ba{q16,  qt16, do16, dot16, k16, v16, kt16, lse2, delta, rows, nt, np, H / G, H,
                   scale * 1.4426950408889634f, scale, dk_part, dv_part, dq, tm, dq_rot};
  if (dq_dtype == CM_F32) {
    hipLaunchKernelGGL(attn_bwd_kernel<float>, dim3(2 * H, n_blocks), dim3(kThreads), 0, s, ba);
  } else {
    hipLaunchKernelGGL(attn_bwd_kernel<_Float16>, dim3(2 * H, n_blocks), dim3(kThreads), 0, s, ba);
  }
  if (int st = cm::launch_status()) return st;
  const DqRope dqr{dq_rot, dq, dq_dtype == CM_F32 ? 1 : 0, H};
  const int reduce_y = G + (dq_rot != nullptr ? H : 0);
#define CM_ATTN_REDUCE(KT, VT)                                                                   \
  hipLaunchKernelGGL((attn_bwd_reduce_kernel<KT, VT>), dim3(np / 8, reduce_y), dim3(256), 0, s,  \
                     dk_part, dv_part, rows, nt, np, H / G, static_cast<KT*>(dk),               \
                     static_cast<VT*>(dv), tm, rope, dqr)
  if (dk_dtype == CM_F32 && dv_dtype == CM_F32) {
    CM_ATTN_REDUCE(float, float);
  } else if (dk_dtype == CM_F16 && dv_dtype == CM_F16) {
    CM_ATTN_REDUCE(_Float16, _Float16);
  } else if (dk_dtype == CM_F16) {
    CM_ATTN_REDUCE(_Float16, float);
  } else {
    CM_ATTN_REDUCE(float, _Float16);
  }
#undef CM_ATTN_REDUCE
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_attn_bwd(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k,
                           int k_dtype, int64_t sk_h, int64_t sk_t, const void* v, int v_dtype,
                           int64_t sv_h, int64_t sv_t, const void* out, const void* dout,
                           const float* lse2, const void* rows_image, int64_t n_tokens,
                           int64_t n_pad, int H, int G, int head_dim, float scale, void* dq,
                           int dq_dtype, void* dk, void* dv, int dkv_dtype,
                           int grads_token_major, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  return bwd_impl(q, q_dtype, sq_h, sq_t, k, k_dtype, sk_h, sk_t, v, v_dtype, sv_h, sv_t,
                  Rope{nullptr, nullptr, 0}, out, dout, lse2, rows_image, n_tokens, n_pad, H, G,
                  head_dim, scale, dq, dq_dtype, dk, dkv_dtype, dv, dkv_dtype, grads_token_major,
                  workspace, workspace_bytes, stream);
}

extern "C" int cm_attn_bwd_rope(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t,
                                const void* k, int k_dtype, int64_t sk_h, int64_t sk_t,
                                const void* v, int v_dtype, int64_t sv_h, int64_t sv_t,
                                const float* cos, const float* sin, int64_t cs_t,
                                const void* out, const void* dout, const float* lse2,
                                const void* rows_image, int64_t n_tokens, int64_t n_pad, int H,
                                int G, int head_dim, float scale, void* dq, int dq_dtype,
                                void* dk, int dk_dtype, void* dv, int dv_dtype,
                                int grads_token_major, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  CM_CHECK_ARG(cos != nullptr);
  return bwd_impl(q, q_dtype, sq_h, sq_t, k, k_dtype, sk_h, sk_t, v, v_dtype, sv_h, sv_t,
                  Rope{cos, sin, cs_t}, out, dout, lse2, rows_image, n_tokens, n_pad, H, G,
                  head_dim, scale, dq, dq_dtype, dk, dk_dtype, dv, dv_dtype, grads_token_major,
                  workspace, workspace_bytes, stream);
}
