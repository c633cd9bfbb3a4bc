// fp16 "NT" GEMM core on the gfx950 matrix cores with direct global -> LDS loads:
// C[m][n] = sum_k A[m][k] B[n][k], fp32 accumulation in v_mfma_f32_32x32x16_f16 tiles, the
// accumulators handed to an epilogue functor.
//
// Operand tiles travel HBM/L2 -> LDS through global_load_lds_dwordx4: the data never passes
// through VGPRs, so the load path costs one issue slot per 16 bytes and no registers. Each
// such instruction writes 64 consecutive 16-byte LDS slots (M0 base + 16 * lane); the XOR
// swizzle of the LDS rows (swz()) is therefore applied on the global side: the lane that owns
// LDS slot (row, physical chunk) fetches logical chunk physical ^ swz(row) of that row.
// Chunks outside the operands (rows past the end, columns past k_len) are fetched from a
// 16-byte zero block instead, so edge tiles need no separate path (hidden sizes are multiples
// of 8, so a 16-byte chunk is either wholly inside or wholly outside).
//
// The LDS holds a ring of S stages of BK (64 or 32) columns; stages kt + 1 .. kt + S - 1 are in
// flight while stage kt is multiplied. One barrier per stage: after it every wavefront has finished reading stage
// kt - 1 (so its buffer can be refilled) and every wavefront's loads of stage kt have landed.
//
// An A-fragment transform FX may rescale each 8-element A fragment between the LDS read and the
// MFMA (used by the LM head's gradient GEMM to turn stored e^{z - m} into probabilities). The
// epilogue's prepare() runs before the main loop (to issue its own loads early), start() gives
// the accumulators their initial values (it may issue loads) and started() runs after the
// prologue's loads; apply() receives the accumulators and the LDS ring, which it may reuse
// after a barrier. ZeroStart is the plain start (zero accumulators).
#pragma once

#include <type_traits>

#include "common.h"
#include "gemm_nt.h"

namespace cm {
namespace gemm {

// Source of the chunks that lie outside an operand.
static __device__ const uint4 kZeroChunk[1] = {{0u, 0u, 0u, 0u}};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One global_load_lds_dwordx4: 64 lanes x 16 bytes into 64 consecutive 16-byte LDS slots from
// lds_slot0 (wave-uniform, passed in M0). Issued through inline assembly: the compiler models the
// builtin like a FLAT access that may complete out of order with LDS reads, and then turns every
// later fragment wait into lgkmcnt(0), which ties the LDS reads of each substep to the freshly
// issued ds_reads. Completion of these loads is waited for explicitly (wait_vmcnt before the
// stage barrier); a counter the compiler does not know about can only make its own waits
// longer, never shorter.
// M0 is set inside the statement; no other code in these kernels keeps a value in M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint4* lds_slot0) {
  const uint32_t m0v = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)lds_slot0));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(m0v), "v"(g)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS operand tiles of ROWS rows x BK fp16 columns = BK / 8 chunks of 16 bytes per row, in one of
// two layouts, chosen per operand by its source layout (Src::kChunkMajor):
//  - row-major (CM = false): slot row * kRC + (chunk ^ swz(row)). The XOR swizzle is chosen for
//    the 64 banks of 4 bytes of the gfx950 LDS: a ds_read_b128 is served 16 lanes (256 bytes)
//    at a time, and the 16 lanes of a fragment read are 16 consecutive rows at one logical
//    chunk, so those rows must land in 16 distinct 16-byte bank groups. With 8-chunk rows the
//    row parity already picks the half of the 256-byte bank span and (row >> 1) & 7 the chunk;
//    with 4-chunk rows row & 3 picks the quarter and (row >> 2) & 3 the chunk. A wavefront's
//    direct load then fetches 8 rows x 128 bytes, the right shape for row-contiguous sources.
//  - chunk-major (CM = true): slot chunk * ROWS + row. A fragment read's 16 rows are 16
//    consecutive slots (conflict-free with no swizzle), and a wavefront's direct load fetches 64
//    consecutive rows at one chunk: two 512-byte spans of a Tiled32 source.
template <int BK, bool CM, int ROWS>
struct LdsTile {
  static constexpr int kRC = BK / 8;
  static_assert(kRC == 8 || kRC == 4, "stages of 64 or 32 columns");
  static __device__ __forceinline__ int swz(int row) {
    return kRC == 8 ? ((row >> 1) & 7) : ((row >> 2) & 3);
  }
  static __device__ __forceinline__ int slot(int row, int ch) {
    return CM ? ch * ROWS + row : row * kRC + (ch ^ swz(row));
  }
  static __device__ __forceinline__ half8 frag(const uint4* lds, int row, int ch) {
    return __builtin_bit_cast(half8, lds[slot(row, ch)]);
  }
};

// The row-major layout on its own (its slots do not depend on the tile's row count).
template <int BK>
using LdsRows = LdsTile<BK, false, 0>;

// Direct loads of one ROWS x BK operand tile by NW wavefronts. Instruction i of a lane fills
// LDS slot (i * NW + wave) * 64 + lane of the tile. Row-major: row row0 + i * kRowStep and (with
// NW >= 2) the same swizzled column for every i, since kRowStep is a multiple of the swizzle's
// period. Chunk-major: row row0 and column col0 + 8 i * kColStep. Either way a lane keeps one
// byte offset from the stage origin, and instruction i adds i times a wave-uniform step; a
// stage's origin is a wave-uniform pointer. Tiles that are wholly inside the operand take that
// path; the others select the zero chunk per lane.
template <int ROWS, int NW, int BK, bool CM = false>
struct DmaTile {
  using L = LdsTile<BK, CM, ROWS>;
  static constexpr int kChunks = ROWS * L::kRC;
  static constexpr int kPer = kChunks / (NW * kWave);  // instructions per lane
  static constexpr int kRowStep = CM ? 0 : NW * kWave / L::kRC;  // tile rows between them
  static constexpr int kColStep = CM ? NW * kWave / ROWS : 0;    // chunks between them
  static_assert(kPer * NW * kWave == kChunks, "tile chunks must split over the wavefronts");
  static_assert(CM || NW >= 2, "one swizzled column per lane needs a row step of 16 or more");
  static_assert(!CM || kColStep * ROWS == NW * kWave, "an instruction covers whole chunk columns");
  uint32_t off0;      // byte offset of the lane's chunk of instruction 0 from the stage origin
  uint32_t step;      // bytes between instructions (wave-uniform)
  int row0, col0;     // tile row and column of the lane's chunk of instruction 0

  template <class Src>
  __device__ __forceinline__ void init(const Src& src, int wave, int lane) {
    const int c = wave * kWave + lane;
    if (CM) {
      row0 = c % ROWS;
      col0 = (c / ROWS) * 8;
      step = src.tile_offset(0, kColStep * 8);
    } else {
      row0 = c / L::kRC;
      col0 = ((c % L::kRC) ^ L::swz(row0)) * 8;
      step = src.tile_offset(kRowStep, 0);
    }
    off0 = src.tile_offset(row0, col0);
  }

  // Instruction i of the stage whose origin is (r0, k0), for a tile known to lie wholly inside
  // the operand: no bounds selection.
  template <class Src>
  __device__ __forceinline__ void issue_inside(const Src& src, int r0, int k0, uint4* tile,
                                               int wave, int i) const {
    const char* base = reinterpret_cast<const char*>(src.at(r0, k0));
    dma16(base + off0 + i * step, tile + (i * NW + wave) * kWave);
  }

  // Instruction i of the stage whose origin is (r0, k0); `inside` = the tile is wholly inside
  // the operand (one wave-uniform test per stage).
  template <class Src>
  __device__ __forceinline__ void issue(const Src& src, int r0, int k0, uint4* tile, int wave,
                                        int i, bool inside) const {
    const char* base = reinterpret_cast<const char*>(src.at(r0, k0));
    const int row = row0 + i * kRowStep, col = col0 + i * kColStep * 8;
    const bool ok = inside || (r0 + row < src.rows && src.col_ok(k0 + col));
    const void* g = ok ? static_cast<const void*>(base + off0 + i * step)
                       : static_cast<const void*>(kZeroChunk);
    dma16(g, tile + (i * NW + wave) * kWave);
  }
};

// Direct loads of a k-major operand (KMajor): the LDS tile is BK rows (k) of BN fp16 (n), row by
// row, with the 32-byte segments of a row XOR-swizzled by kswz(k) = 2 ((k >> 1) & 1) within
// aligned groups of four segments. A transposing fragment read (frag_kmajor) has its 16-lane
// groups read rows k .. k + 3 (k a multiple of 4) at one 32-byte segment and the next, so with
// this swizzle the 8 (row, segment) pieces a 32-lane half serves at once cover the 64 banks
// exactly once. Instruction i of a lane fills slot c = (i NW + wave) 64 + lane of the tile: row
// c / (BN / 8), physical slot c % (BN / 8); the slot positions differ per instruction, so the
// lane keeps one byte offset per instruction.
template <int BN, int NW, int BK>
struct DmaTileK {
  static constexpr int kSlotsRow = BN / 8;
  static constexpr int kChunks = BK * kSlotsRow;
  static constexpr int kPer = kChunks / (NW * kWave);
  static_assert(kPer * NW * kWave == kChunks, "tile chunks must split over the wavefronts");
  static_assert(BN % 64 == 0, "rows of whole groups of four 32-byte segments");
  static __device__ __forceinline__ int kswz(int k) { return ((k >> 1) & 1) * 2; }
  uint32_t off[kPer];  // byte offset of the lane's chunk of instruction i from the stage origin
  int krow[kPer], ncol[kPer];

  template <class Src>
  __device__ __forceinline__ void init(const Src& src, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = (i * NW + wave) * kWave + lane;
      const int k = c / kSlotsRow, ps = c % kSlotsRow;
      const int ls = (((ps >> 1) ^ kswz(k)) << 1) | (ps & 1);  // logical slot of the row
      krow[i] = k;
      ncol[i] = ls * 8;
      off[i] = static_cast<uint32_t>((static_cast<int64_t>(k) * src.ld + ncol[i]) * 2);
    }
  }
  template <class Src>
  __device__ __forceinline__ void issue_inside(const Src& src, int n0, int k0, uint4* tile,
                                               int wave, int i) const {
    const char* base = reinterpret_cast<const char*>(src.at(n0, k0));
    dma16(base + off[i], tile + (i * NW + wave) * kWave);
  }
  template <class Src>
  __device__ __forceinline__ void issue(const Src& src, int n0, int k0, uint4* tile, int wave,
                                        int i, bool inside) const {
    const char* base = reinterpret_cast<const char*>(src.at(n0, k0));
    const bool ok = inside || (k0 + krow[i] < src.k_len && n0 + ncol[i] < src.rows);
    const void* g = ok ? static_cast<const void*>(base + off[i])
                       : static_cast<const void*>(kZeroChunk);
    dma16(g, tile + (i * NW + wave) * kWave);
  }
};

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4_t;

// The B fragment of v_mfma_f32_32x32x16_f16 (lane l: n = l % 32 of the 32-column tile at n_base,
// k = ks * 16 + (l / 32) * 8 .. + 7) from a k-major LDS tile of BN columns, as two
// ds_read_b64_tr_b16. That instruction (lane layout checked on the box) gives lane i of each
// 16-lane group element i % 4 of the 8 bytes that lane 4 j + i / 4 of the group addressed, for
// j = 0 .. 3: so lane a of group g addresses row k0 + a / 4, columns n_base + 16 (g % 2) +
// 4 (a % 4) .. + 3, and lane i receives rows k0 .. k0 + 3 of column n_base + 16 (g % 2) + i.
template <int BN>
__device__ __forceinline__ half8 frag_kmajor(const uint4* tile, int n_base, int ks, int lane) {
  const int g = lane / 16, a = lane % 16;
  const int n = n_base + (g % 2) * 16 + 4 * (a % 4);
  const int k = ks * 16 + (g / 2) * 8 + a / 4;
  const int seg = (n / 16) ^ DmaTileK<BN, 1, 16>::kswz(k);  // kswz(k + 4) == kswz(k)
  const char* row = reinterpret_cast<const char*>(tile) + k * (BN * 2) + seg * 32 + (n % 16) * 2;
  const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(row));
  const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(row + 4 * BN * 2));
  const short4v v[2] = {lo, hi};
  return __builtin_bit_cast(half8, v);
}

// Workgroup barrier that orders LDS only: the loads into LDS are waited for explicitly
// (vmcnt), so the barrier must not wait for every outstanding global load.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Accumulators starting at zero, for epilogues with nothing to add to the product.
struct ZeroStart {
  template <int TM, int TN>
  static __device__ __forceinline__ void start(floatx16 (&acc)[TM][TN], int, int, int) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }
  template <int TM, int TN>
  static __device__ __forceinline__ void started(floatx16 (&)[TM][TN]) {}
};

// Identity A-fragment transform with no per-stage data (the default FX of gemm_lds). An FX
// provides bind(row) (the A row of the calling lane's fragment 0; fragment i is row + 32 i),
// prefetch(k0) (register loads for the stage at column k0, issued one stage ahead),
// advance() (the prefetched values become current) and apply(frag, i) on the A fragment of the
// wavefront's tile row i.
struct PlainA {
  __device__ __forceinline__ void bind(int) {}
  __device__ __forceinline__ void prefetch(int) {}
  __device__ __forceinline__ void advance() {}
  __device__ __forceinline__ half8 apply(half8 f, int) const { return f; }
};

// Main loop, per stage kt: wait until stage kt has landed and this wavefront's fragment reads of
// stage kt - 1 have returned, one barrier (stage kt visible; every wavefront is done with stage
// kt - 1, whose buffer is refilled next), then five MFMA groups: the last substep of stage
// kt - 1 (its fragments are already in registers, so these MFMAs cover the latency of the first
// fragment reads of stage kt), then substeps 0 .. KS - 2 of stage kt, each after the reads of the
// next substep's fragments. Each group issues its share of the loads of stage kt + S - 1 between
// its two halves. Spreading the LDS-direct loads between MFMAs keeps the texture unit's queue
// short, so a wavefront never stalls in issue with the matrix core idle (issued as one burst
// after the barrier, the loads of a 256 x 256 x 64 stage held every wavefront for ~1000
// cycles). sched_barrier pins that order.
// Bounds handling of the operand loads (EDGE): kEdgeEither picks per workgroup (a second copy of
// the main loop without bounds selection, taken when every stage lies inside both operands),
// kEdgeAlways always selects, kEdgeNever never does (the caller guarantees every tile of the
// launch lies inside: one loop, for kernels where two copies would not fit the registers).
enum EdgeMode { kEdgeEither = 0, kEdgeAlways = 1, kEdgeNever = 2 };

template <int BM, int BN, int WM, int WN, int BK, int S, class SrcA, class SrcB, class Epi,
          class FX = PlainA, int EDGE = kEdgeEither>
__device__ __forceinline__ void gemm_lds(const SrcA& A, const SrcB& B, int k_begin, int k_end,
                                         int tm, int tn, Epi& epi, uint4* lds, FX fx = FX()) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  using LA = LdsTile<BK, SrcA::kChunkMajor, BM>;
  using LB = LdsTile<BK, SrcB::kChunkMajor, BN>;
  constexpr int KS = BK / 16;  // MFMA substeps per stage
  static_assert(TM * 32 == WTM && TN * 32 == WTN, "wave tiles are multiples of 32");
  static_assert(S >= 2, "at least a double buffer");
  constexpr int kStage = (BM + BN) * LA::kRC;  // uint4 per stage
  using TA = DmaTile<BM, NW, BK, SrcA::kChunkMajor>;
  static_assert(!SrcA::kKMajor, "a k-major operand is B");
  using TB = std::conditional_t<SrcB::kKMajor, DmaTileK<BN, NW, BK>,
                                DmaTile<BN, NW, BK, SrcB::kChunkMajor>>;
  constexpr int kDma = TA::kPer + TB::kPer;     // LDS-direct loads per lane per stage
  constexpr int kPart = (kDma + KS - 1) / KS;   // of them issued per substep
  constexpr int kHalf = (TM * TN) / 2;          // MFMAs before the loads of a substep
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave / WN, wn = wave % WN;
  TA la;
  TB lb;
  la.init(A, wave, lane);
  lb.init(B, wave, lane);
  epi.template prepare<TM, TN>(m0 + wm * WTM, n0 + wn * WTN, lane);

  // The epilogue's start() sets the accumulators (zero, or loads issued here so that they are
  // in flight with the first stage's loads); started() runs once the first stage has landed.
  floatx16 acc[TM][TN];
  epi.template start<TM, TN>(acc, m0 + wm * WTM, n0 + wn * WTN, lane);

  const int n_kt = (k_end - k_begin + BK - 1) / BK;
  auto inside_a = [&](int kt) { return A.tile_inside(m0, BM, k_begin + kt * BK); };
  auto inside_b = [&](int kt) { return B.tile_inside(n0, BN, k_begin + kt * BK); };
  // Every stage of the workgroup's tiles lies inside both operands (the common case: the
  // bounds tests are monotonic in the stage, so the last stage decides); the main loop then
  // issues its loads with no bounds selection.
  const bool all_inside = n_kt > 0 && inside_a(n_kt - 1) && inside_b(n_kt - 1);
  // load instruction q (< kDma) of stage kt: A's instructions first, then B's
  auto issue = [&](int kt, int q, bool in_a, bool in_b, auto edge) {
    uint4* st = lds + (kt % S) * kStage;
    const int k0 = k_begin + kt * BK;
    if (q < TA::kPer) {
      if constexpr (decltype(edge)::value) la.issue(A, m0, k0, st, wave, q, in_a);
      else la.issue_inside(A, m0, k0, st, wave, q);
    } else {
      if constexpr (decltype(edge)::value) lb.issue(B, n0, k0, st + BM * LA::kRC, wave, q - TA::kPer, in_b);
      else lb.issue_inside(B, n0, k0, st + BM * LA::kRC, wave, q - TA::kPer);
    }
  };
  const int arow = wm * WTM + lane % 32, brow = wn * WTN + lane % 32;
  half8 af[2][TM], bf[2][TN];
  auto read = [&](int kt, int ks, int buf) {
    const uint4* As = lds + (kt % S) * kStage;
    const uint4* Bs = As + BM * LA::kRC;
    const int ch = ks * 2 + lane / 32;
#pragma unroll
    for (int i = 0; i < TM; ++i) af[buf][i] = fx.apply(LA::frag(As, arow + i * 32, ch), i);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (SrcB::kKMajor) {
        bf[buf][j] = frag_kmajor<BN>(Bs, wn * WTN + j * 32, ks, lane);
      } else {
        bf[buf][j] = LB::frag(Bs, brow + j * 32, ch);
      }
    }
  };
  // Scheduling of a group "fragment reads of the next substep + first half of the MFMAs":
  // one LDS read, one MFMA, alternately (measured 1.5% faster on the LM head than all reads
  // first).
  constexpr int kReads = TM + (SrcB::kKMajor ? 2 : 1) * TN;  // LDS reads per substep
  auto interleave_reads = [] {
#pragma unroll
    for (int i = 0; i < (kReads > kHalf ? kReads : kHalf); ++i) {
      if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if (i < kHalf) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
    }
  };
  auto mfma = [&](int b, int g0, int g1) {
#pragma unroll
    for (int g = g0; g < g1; ++g) {
      const int i = g / TN, j = g % TN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[b][i], bf[b][j], acc[i][j], 0, 0, 0);
    }
  };

  // Prologue: stages 0 .. S - 2 in flight (the FX prefetch of stage 0 first).
  fx.bind(m0 + wm * WTM + lane % 32);
  if (n_kt > 0) fx.prefetch(k_begin);
#pragma unroll
  for (int s = 0; s < S - 1; ++s) {
    if (s < n_kt) {
      const bool ia = inside_a(s), ib = inside_b(s);
#pragma unroll
      for (int q = 0; q < kDma; ++q) issue(s, q, ia, ib, std::true_type{});
    }
  }

  // Waits for the prologue's loads (the first stage and whatever start() issued).
  epi.template started<TM, TN>(acc);

  // Stage kt. The last substep of stage kt - 1 is multiplied after the barrier of stage kt: its
  // fragments are already in registers, so its MFMAs cover the latency of the first fragment
  // reads of stage kt. Before the barrier each wavefront waits for its own reads (the buffer they
  // read from is refilled after it). The bounds selection on the loads is compile-time (EDGE):
  // with kEdgeEither a workgroup whose every stage lies inside both operands runs a copy of the
  // loop without it. (Peeling the first stage and the load-free last stages as well, or two loop
  // copies in the LM head's gradient GEMM, pushed it past 256 registers.)
  static_assert(KS % 2 == 0, "substep buffers alternate within a stage");
  auto run = [&](auto edge) {
    for (int kt = 0; kt < n_kt; ++kt) {
      if (kt + S - 2 < n_kt) {
        wait_vmcnt<(S - 2) * kDma>();
      } else {
        wait_vmcnt<0>();
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own fragment reads have landed
      lds_barrier();
      fx.advance();
      if (kt + 1 < n_kt) fx.prefetch(k_begin + (kt + 1) * BK);
      const int kl = kt + S - 1;
      const bool load = kl < n_kt;
      bool ia = true, ib = true;
      if constexpr (decltype(edge)::value) {
        ia = load && inside_a(kl);
        ib = load && inside_b(kl);
      }
      read(kt, 0, 0);
      if (kt > 0) {
        mfma(1, 0, kHalf);
        interleave_reads();
      }
      __builtin_amdgcn_sched_barrier(0);
      if (load) {
#pragma unroll
        for (int q = 0; q < kPart; ++q)
          if (q < kDma) issue(kl, q, ia, ib, edge);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kt > 0) mfma(1, kHalf, TM * TN);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks + 1 < KS; ++ks) {
        const int b = ks & 1;
        read(kt, ks + 1, b ^ 1);
        mfma(b, 0, kHalf);
        interleave_reads();
        __builtin_amdgcn_sched_barrier(0);
        if (load) {
#pragma unroll
          for (int q = (ks + 1) * kPart; q < (ks + 2) * kPart; ++q)
            if (q < kDma) issue(kl, q, ia, ib, edge);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma(b, kHalf, TM * TN);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if constexpr (EDGE == kEdgeEither) {
    if (all_inside) {
      run(std::false_type{});
    } else {
      run(std::true_type{});
    }
  } else {
    (void)all_inside;
    run(std::bool_constant<EDGE == kEdgeAlways>{});
  }
  if (n_kt > 0) mfma(1, 0, TM * TN);
  epi.template apply<TM, TN>(acc, m0 + wm * WTM, n0 + wn * WTN, lane, lds);
}

}  // namespace gemm
}  // namespace cm
