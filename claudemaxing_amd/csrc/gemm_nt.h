// Operand layouts of the fp16 "NT" GEMMs on the gfx950 matrix cores (C[m][n] = sum_k A[m][k]
// B[n][k], both operands K-contiguous), the MFMA register types, and the workgroup -> tile map.
//   RowMajor  element (r, k) at p[r * ld + k];
//   Blocked64 element (r, k) at p[((k / 64) * rows + r) * 64 + k % 64], i.e. 64-column panels,
//             so a (rows x 64) tile of one panel is a single contiguous span. Panels are padded
//             to 64 columns (the padding must hold finite values; the LM head keeps zeros there).
//   Tiled32   32-row x 64-column blocks of 8-column chunks (below);
//   KMajor    the operand stored transposed, [K][N] with N contiguous (below).
// The main loop that consumes them is in gemm_lds.h.
#pragma once

#include "common.h"

namespace cm {
namespace gemm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;              // K elements per stage
constexpr int kRowChunks = kBK / 8;  // 16-byte chunks per tile row

struct RowMajor {
  static constexpr bool kChunkMajor = false;  // LDS tile layout (gemm_lds.h)
  static constexpr bool kKMajor = false;
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
  // bytes from element (r0, k0) to (r0 + r, k0 + k) of a tile (k < 64)
  __device__ __forceinline__ uint32_t tile_offset(int r, int k) const {
    return static_cast<uint32_t>((static_cast<int64_t>(r) * ld + k) * 2);
  }
};

struct Blocked64 {
  static constexpr bool kChunkMajor = false;
  static constexpr bool kKMajor = false;
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
  // bytes from element (r0, k0) to (r0 + r, k0 + k) of a tile (k0 a multiple of 64, k < 64)
  __device__ __forceinline__ uint32_t tile_offset(int r, int k) const {
    return static_cast<uint32_t>((r * kBK + k) * 2);
  }
};

// 4 KiB blocks of 32 rows x 64 columns, 8-column chunks inside: element (r, k) at
// p[(((k / 64) * row_blocks + r / 32) * 8 + (k % 64) / 8) * 256 + (r % 32) * 8 + k % 8], with
// row_blocks = ceil(rows / 32). One 16-byte chunk is 8 consecutive columns of a row, and the
// chunks of 32 consecutive rows at one 8-column position are one 512-byte span, so a producer
// whose lanes hold consecutive rows (the LM head's logits epilogue: one token per lane) writes
// whole spans straight from registers, while a GEMM stage's 8-row x 64-column slices stay inside
// one block. As with Blocked64, the columns up to the end of the last 64-column panel must hold
// finite values.
struct Tiled32 {
  static constexpr bool kChunkMajor = true;
  static constexpr bool kKMajor = false;
  const _Float16* p;
  int rows;        // valid rows
  int k_len;       // columns
  int row_blocks;  // ceil(rows / 32)
  static __host__ __device__ __forceinline__ int64_t index(int64_t r, int64_t k, int row_blocks) {
    return (((k / 64) * row_blocks + r / 32) * 8 + (k % 64) / 8) * 256 + (r % 32) * 8 + k % 8;
  }
  __device__ __forceinline__ const _Float16* at(int r, int k) const {
    return p + index(r, k, row_blocks);
  }
  __device__ __forceinline__ bool tile_inside(int r0, int n_rows, int k0) const {
    return r0 + n_rows <= rows && k0 < k_len;
  }
  __device__ __forceinline__ bool col_ok(int k) const { return (k / kBK) * kBK < k_len; }
  // bytes from element (r0, k0) to (r0 + r, k0 + k) of a tile (r0 a multiple of 32, k0 of 64,
  // k < 64 a multiple of 8)
  __device__ __forceinline__ uint32_t tile_offset(int r, int k) const {
    return static_cast<uint32_t>(((r / 32) * 8 + k / 8) * 512 + (r % 32) * 16);
  }
};

// An NT operand stored transposed, [K][N] with N contiguous: element (row n, column k) of the
// operand at p[k * ld + n]. The LM head reads its weight W [V][H] this way as the gradient GEMM's
// B operand (rows = hidden units, K = vocabulary), so that no transposed copy of W is needed.
// Its LDS tiles are k-major and its MFMA fragments are assembled by transposing LDS reads
// (gemm_lds.h, DmaTileK and frag_kmajor).
struct KMajor {
  static constexpr bool kChunkMajor = false;
  static constexpr bool kKMajor = true;
  const _Float16* p;
  int64_t ld;  // elements between consecutive k
  int rows;    // valid n
  int k_len;   // valid k
  __device__ __forceinline__ const _Float16* at(int n, int k) const {
    return p + static_cast<int64_t>(k) * ld + n;
  }
  __device__ __forceinline__ bool tile_inside(int n0, int n_rows, int k0) const {
    return n0 + n_rows <= rows && k0 + kBK <= k_len;
  }
};

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

// The same for block `bid` of `count` blocks of one role inside a larger grid (the caller keeps
// bid % 8 equal to the block's XCD). remap requires count % 8 == 0.
__device__ __forceinline__ void tile_of(int bid, int count, int tiles_n, int remap, int& tm,
                                        int& tn) {
  if (remap) bid = (bid % 8) * (count / 8) + bid / 8;
  tm = bid / tiles_n;
  tn = bid % tiles_n;
}

// Split-K form of tile_of: `count` = tiles * slices blocks; each XCD gets a contiguous range of
// (slice, tile) ids, i.e. one K-slice and a block of tile rows.
__device__ __forceinline__ void tile_of_sliced(int bid, int count, int tiles, int tiles_n,
                                               int remap, int& tm, int& tn, int& slice) {
  if (remap) bid = (bid % 8) * (count / 8) + bid / 8;
  slice = bid / tiles;
  const int t = bid % tiles;
  tm = t / tiles_n;
  tn = t % tiles_n;
}

// The same over a 2-D grid (blockIdx.y = K-slice): the flattened (slice, tile) ids are laid out
// so that each XCD gets a contiguous range, i.e. one K-slice and a block of tile rows, whose
// operand tiles its L2 then shares. remap requires gridDim.x * gridDim.y % 8 == 0.
__device__ __forceinline__ void tile_of_block_2d(int tiles_n, int remap, int& tm, int& tn,
                                                 int& slice) {
  const int total = gridDim.x * gridDim.y;
  int bid = blockIdx.x + blockIdx.y * gridDim.x;
  if (remap) bid = (bid % 8) * (total / 8) + bid / 8;
  slice = bid / gridDim.x;
  const int t = bid % gridDim.x;
  tm = t / tiles_n;
  tn = t % tiles_n;
}

}  // namespace gemm
}  // namespace cm
