// fp16 "NT" GEMM core on the gfx950 matrix cores: C[m][n] = sum_k A[m][k] B[n][k], fp32
// accumulation in v_mfma_f32_32x32x16_f16 tiles, the accumulators handed to an epilogue functor.
//
// Operands are K-contiguous and come in two layouts:
//   RowMajor  element (r, k) at p[r * ld + k];
//   Blocked64 element (r, k) at p[((k / 64) * rows + r) * 64 + k % 64], i.e. 64-column panels,
//             so a (rows x 64) tile of one panel is a single contiguous span. Panels are padded
//             to 64 columns (the padding must hold finite values; the LM head keeps zeros there).
// A workgroup has WM x WN wavefronts (4 or 8). Each pipeline stage moves a BM x 64 tile of A and
// a BN x 64 tile of B global -> registers -> LDS with 16-byte accesses. Tiles entirely inside the matrices take a branch-free path (one
// scalar test per tile); edge tiles fall back to per-element bounds checks. LDS rows of 64 fp16
// (128 B = 8 chunks of 16 B) are XOR-swizzled so that the fragment reads of a wavefront do not
// collide on LDS banks (see swz()). With STAGES = 2 the LDS is double-buffered (one barrier per
// stage, the next stage's global loads overlap this stage's MFMAs); with STAGES = 1 a single LDS
// buffer halves the footprint so that two workgroups share a CU.
#pragma once

#include "common.h"

namespace cm {
namespace gemm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;              // K elements per stage
constexpr int kRowChunks = kBK / 8;  // 16-byte chunks per tile row

// LDS swizzle: physical 16-byte chunk = logical chunk ^ swz(row). With SHIFT = 0 eight
// consecutive rows use eight distinct chunks (all 32 banks of a 128-byte span); SHIFT = 1 pairs
// rows instead (distinct banks for 16 rows of a 64-bank view). Measured on MI355X for the LM
// head GEMMs, SHIFT = 0 is faster although the bank-conflict counter reads higher.
#ifndef CM_SCHED_HINTS
#define CM_SCHED_HINTS 0
#endif
#ifndef CM_SWZ_SHIFT
#define CM_SWZ_SHIFT 0
#endif
__device__ __forceinline__ int swz(int row) { return (row >> CM_SWZ_SHIFT) & 7; }

struct RowMajor {
  const _Float16* p;
  int64_t ld;
  int rows;   // valid rows
  int k_len;  // valid columns
  __device__ __forceinline__ const _Float16* at(int r, int k) const {
    return p + static_cast<int64_t>(r) * ld + k;
  }
  __device__ __forceinline__ bool tile_inside(int r0, int n_rows, int k0) const {
    return r0 + n_rows <= rows && k0 + kBK <= k_len;
  }
  __device__ __forceinline__ bool col_ok(int k) const { return k < k_len; }
};

struct Blocked64 {
  const _Float16* p;
  int rows;   // valid rows (= rows of a panel)
  int k_len;  // columns, padded panels beyond it hold finite values
  __device__ __forceinline__ const _Float16* at(int r, int k) const {
    return p + ((static_cast<int64_t>(k / kBK) * rows + r) * kBK + k % kBK);
  }
  __device__ __forceinline__ bool tile_inside(int r0, int n_rows, int k0) const {
    return r0 + n_rows <= rows && k0 < k_len;
  }
  // the panel holding k exists (padding columns are read as stored)
  __device__ __forceinline__ bool col_ok(int k) const { return (k / kBK) * kBK < k_len; }
};

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// Identity operand transform (tile data goes to LDS unchanged).
struct NoXform {
  __device__ __forceinline__ void prepare(int, int) {}
  __device__ __forceinline__ void apply(uint4&, int) const {}
};
// An A transform X sees chunk i of the calling thread (tile row (threadIdx.x + i THREADS) / 8)
// through X::apply(chunk, i); X::prepare(m0, tile_rows) runs once per workgroup.

template <int ROWS, int THREADS>
struct TileLoad {
  static constexpr int kPer = ROWS * kRowChunks / THREADS;
  static_assert(kPer * THREADS == ROWS * kRowChunks, "tile rows must split over the threads");
  uint4 v[kPer];

  // Row of the tile that chunk i of this thread belongs to.
  static __device__ __forceinline__ int row_of(int i) {
    return (threadIdx.x + i * THREADS) / kRowChunks;
  }

  template <class Src>
  __device__ __forceinline__ void load(const Src& src, int r0, int k0) {
    if (src.tile_inside(r0, ROWS, k0)) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int c = threadIdx.x + i * THREADS;
        v[i] = *reinterpret_cast<const uint4*>(src.at(r0 + c / kRowChunks,
                                                      k0 + (c % kRowChunks) * 8));
      }
    } else {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int c = threadIdx.x + i * THREADS;
        const int r = r0 + c / kRowChunks;
        const int k = k0 + (c % kRowChunks) * 8;
        if (r < src.rows && src.col_ok(k) && src.col_ok(k + 7)) {
          v[i] = *reinterpret_cast<const uint4*>(src.at(r, k));
        } else if (r < src.rows && src.col_ok(k)) {
          union {
            uint4 u;
            _Float16 h[8];
          } t;
#pragma unroll
          for (int e = 0; e < 8; ++e) t.h[e] = src.col_ok(k + e) ? *src.at(r, k + e) : _Float16(0);
          v[i] = t.u;
        } else {
          v[i] = zero4();
        }
      }
    }
  }

  template <class X>
  __device__ __forceinline__ void transform(const X& x) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) x.apply(v[i], i);
  }

  __device__ __forceinline__ void store(uint4* lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * THREADS;
      const int row = c / kRowChunks;
      lds[row * kRowChunks + ((c % kRowChunks) ^ swz(row))] = v[i];
    }
  }
};

__device__ __forceinline__ half8 frag(const uint4* lds, int row, int ch) {
  return __builtin_bit_cast(half8, lds[row * kRowChunks + (ch ^ swz(row))]);
}

// Workgroup -> (tile_m, tile_n), tile_n fastest. With remap (grid a multiple of 8), logical tile
// ids are laid out so that consecutive ones run on the same XCD (hardware dispatches workgroup
// ids round-robin over the 8 XCDs), so workgroups that share operand tiles share an L2.
__device__ __forceinline__ void tile_of_block(int tiles_n, int remap, int& tm, int& tn) {
  int bid = blockIdx.x;
  if (remap) {
    const int per = gridDim.x / 8;
    bid = (bid % 8) * per + bid / 8;
  }
  tm = bid / tiles_n;
  tn = bid % tiles_n;
}

// acc[mt][nt][r] of wavefront (wm, wn) holds
//   row m = m0 + wm * BM/WM + 32 mt + 8 (r / 4) + 4 (lane / 32) + r % 4
//   col n = n0 + wn * BN/WN + 32 nt + lane % 32
// The K range [k_begin, k_end) is a multiple of 64 except at the end of the operands.
// XA transforms each A tile in registers before it is written to LDS.
template <int BM, int BN, int WM, int WN, int STAGES, class SrcA, class SrcB, class Epi,
          class XA = NoXform>
__device__ __forceinline__ void gemm_body(const SrcA& A, const SrcB& B, int k_begin, int k_end,
                                          int tm, int tn, Epi& epi, uint4* lds,
                                          XA xa = XA()) {
  constexpr int THREADS = WM * WN * kWave;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM * 32 == WTM && TN * 32 == WTN, "wave tiles are multiples of 32");
  constexpr int kStage = (BM + BN) * kRowChunks;  // uint4 per stage
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / WN, wn = wave % WN;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  TileLoad<BM, THREADS> la;
  TileLoad<BN, THREADS> lb;
  xa.prepare(m0, BM);
  la.load(A, m0, k_begin);
  lb.load(B, n0, k_begin);
  la.transform(xa);
  la.store(lds);
  lb.store(lds + BM * kRowChunks);
  __syncthreads();

  const int kt_count = (k_end - k_begin + kBK - 1) / kBK;
  for (int kt = 0; kt < kt_count; ++kt) {
    const int cur = STAGES == 2 ? (kt & 1) : 0;
    const bool more = kt + 1 < kt_count;
    if (more) {
      la.load(A, m0, k_begin + (kt + 1) * kBK);
      lb.load(B, n0, k_begin + (kt + 1) * kBK);
    }
    const uint4* As = lds + cur * kStage;
    const uint4* Bs = As + BM * kRowChunks;
    // Fragments are double-buffered across the four 16-wide K substeps: the LDS reads of
    // substep ks + 1 are issued before the MFMAs of substep ks, so their latency hides behind
    // the matrix work instead of stalling it.
    half8 af[2][TM], bf[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) af[0][i] = frag(As, wm * WTM + i * 32 + lane % 32, lane / 32);
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[0][j] = frag(Bs, wn * WTN + j * 32 + lane % 32, lane / 32);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int b = ks & 1;
      if (ks + 1 < kBK / 16) {
        const int ch = (ks + 1) * 2 + lane / 32;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[b ^ 1][i] = frag(As, wm * WTM + i * 32 + lane % 32, ch);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[b ^ 1][j] = frag(Bs, wn * WTN + j * 32 + lane % 32, ch);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[b][i], bf[b][j], acc[i][j], 0,
                                                             0, 0);
#if CM_SCHED_HINTS
      // interleave: one LDS fragment read between consecutive MFMAs
#pragma unroll
      for (int g = 0; g < TM * TN; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
#endif
    }
    if (more) {
      if (STAGES == 1) __syncthreads();  // every wavefront is done reading the single buffer
      uint4* nxt = lds + (STAGES == 2 ? (cur ^ 1) * kStage : 0);
      la.transform(xa);
      la.store(nxt);
      lb.store(nxt + BM * kRowChunks);
    }
    __syncthreads();
  }
  epi.template apply<TM, TN>(acc, m0 + wm * WTM, n0 + wn * WTN, lane);
}

}  // namespace gemm
}  // namespace cm
