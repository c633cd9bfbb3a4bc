// NF4 weights expanded inside an fp16 GEMM on the gfx950 matrix cores: the dequantization
// (nested absmax included) happens on the way into the LDS, so the fp16 weight never exists
// in HBM.
//
// Replaces, for the frozen 4-bit layers of the training step, the pair "dequantize_nf4 (the
// reference's nf4_dequant_kernel, solution/nf4.py:26-46) -> fp16 GEMM" that the reference's
// patched bitsandbytes matmul runs per linear (solution/nf4.py:102-130, and the recompute in
// solution/swiglu_recompute.py:165-166, 198-199):
//
//   forward   Y_i = X W_i^T (+ b_i)       X fp16 [M, K], W_i NF4 [N_i, K], up to 3 weights that
//                                         share X in one launch (gate + up)
//   backward  dX = sum_i G_i W_i          G_i fp16 [M, N_i], the weights' rows concatenated
//                                         along the contraction (dgate Wg + dup Wu)
//
// Each weight element is expanded exactly as the standalone dequant kernel expands it: scale
// s = code2[absmax8[b]] * absmax2[b / blocksize2] + offset (multiply, then add), value =
// fp16(code[nibble] * s). So a fused product equals the dequant kernel's fp16 weight fed to a
// GEMM, up to the order of the fp32 sums. Outputs are rounded once to fp16 (after the bias, as
// a GEMM with a bias epilogue does) and optionally widened to fp32, which is what "fp16 linear,
// then .to(float32)" gives.
//
// Tiling: C = A B^T on v_mfma_f32_32x32x16_f16 with A = the weight side (BM rows: weight rows
// forward, weight columns backward) and B = the token side (BN tokens). 4 wavefronts in a 2 x 2
// grid; stages of 64 contraction elements, double-buffered in the LDS, one barrier per stage.
// Per stage each lane
//   - issues the direct-to-LDS loads (global_load_lds_dwordx4) of the next token tile,
//   - multiplies the current stage,
//   - expands the next weight tile from the packed bytes it loaded one stage earlier into
//     registers, writing fp16 16-byte (forward) or 8-byte (backward, transposed) LDS chunks,
//   - loads the packed bytes and block scales of the stage after that.
// The forward weight tile is a plain row-major tile; the backward one is the transpose (rows =
// weight columns, contraction = weight rows), assembled from 8 x RPT blocks: each lane loads one
// 4-byte word (8 columns) from RPT consecutive weight rows and writes 8 LDS pieces of RPT
// values. The token side is read as it lies (K-contiguous rows).
#include <type_traits>

#include "common.h"
#include "gemm_lds.h"

namespace {

// The block scale is a multiply then an add, never fused (the dequant kernel's arithmetic).
#pragma clang fp contract(off)

using cm::gemm::DmaTile;
using cm::gemm::floatx16;
using cm::gemm::half8;
using cm::gemm::LdsRows;
using cm::gemm::RowMajor;

constexpr int kThreads = 256;  // 4 wavefronts, 2 x 2
constexpr int kBK = 64;        // contraction elements per stage
constexpr int kMaxW = 3;

struct WeightDev {
  const uint32_t* packed;  // 4-byte words of the packed weight
  const float* smap;       // fp32 block scales [cols / blocksize][rows], or null
  const void* absmax;      // uint8 (nested) or fp32 block scales
  const float* absmax2;
  const float* offset;
  const float* code;       // [16]
  const float* code2;      // [256] (nested)
  int rows;                // N_i
  int bs_shift;            // log2(blocksize)
  int bs2_shift;           // log2(blocksize2), or -1: divide by bs2
  uint32_t bs2;
  int first;               // forward: first A tile; backward: first stage of this weight
  const _Float16* bias;    // forward, may be null
  void* out;               // forward output [M, N_i] (fp16 or fp32)
  int64_t ldo;
  const _Float16* g;       // backward input [M, N_i]
  int64_t ldg;
};

struct Args {
  WeightDev w[kMaxW];
  int n_w;
  int nested;
  int cols;         // K: elements per weight row
  int m;            // tokens
  int tiles_b;      // token tiles
  int remap;        // XCD-aware tile order (grid a multiple of 8)
  int out32;        // outputs widened to fp32
  const _Float16* x;  // forward token operand [M, K]
  int64_t ldx;
  void* dx;         // backward output [M, K]
  int64_t lddx;
  int n_stages;     // backward: total stages over all weights
  // split over the contraction (ws kernel): slices write fp32 partials [split][m][n_out]
  int split;
  float* ws;
  int n_out;        // output columns of the partials
};

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const _Float16 ha = cm::from_f32<_Float16>(a), hb = cm::from_f32<_Float16>(b);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
}

// Block scale of absmax block blk of weight w (the dequant kernel's formula).
__device__ __forceinline__ float block_scale(int nested, float q8code, float a2, float off,
                                             float plain) {
  if (nested) {
    const float prod = q8code * a2;
    return prod + off;
  }
  return plain;
}

// Raw scale inputs of one block, loaded a stage ahead: the u8 code index and absmax2 (nested),
// or the fp32 scale.
struct ScaleRaw {
  uint32_t q8;
  float a2;  // absmax2 (nested) or the fp32 scale
};

__device__ __forceinline__ ScaleRaw load_scale(const WeightDev& w, int nested, int64_t elem) {
  const uint32_t blk = static_cast<uint32_t>(elem >> w.bs_shift);
  ScaleRaw r;
  if (nested) {
    r.q8 = static_cast<const uint8_t*>(w.absmax)[blk];
    const uint32_t b2 = w.bs2_shift >= 0 ? (blk >> w.bs2_shift) : (blk / w.bs2);
    r.a2 = w.absmax2[b2];
  } else {
    r.q8 = 0;
    r.a2 = static_cast<const float*>(w.absmax)[blk];
  }
  return r;
}

// ---------------------------------------------------------------------------------------------
// Weight-side tile loaders. A stage's tile is BM rows x 64 contraction elements in the LDS
// (row-major rows of 8 16-byte chunks, chunk XOR-swizzled by LdsRows<64>::swz(row)).

// Forward: tile rows = weight rows r0 .. r0 + BM, columns kc .. kc + 64. A lane expands EPT =
// BM / 4 consecutive elements of one row (256 lanes), with one block scale per run of up to 32
// elements (blocksize >= 32).
template <int BM>
struct FwdLoader {
  static constexpr int kEPT = BM / 4;             // elements per lane per stage
  static constexpr int kWords = kEPT / 8;         // 4-byte packed words per lane
  static constexpr int kTPR = kBK / kEPT;         // lanes per tile row
  static constexpr int kRuns = kEPT > 32 ? kEPT / 32 : 1;  // block-scale runs per lane
  static_assert(kWords == 2 || kWords == 4 || kWords == 8, "BM of 64, 128 or 256");
  uint32_t word[kWords];
  ScaleRaw sc[kRuns];
  int row, part;

  __device__ __forceinline__ void init(int tid) {
    row = tid / kTPR;
    part = tid % kTPR;
  }
  __device__ __forceinline__ void load(const WeightDev& w, int nested, int cols, int r0, int kc) {
    const int64_t e0 = static_cast<int64_t>(r0 + row) * cols + kc + part * kEPT;
    const uint32_t* p = w.packed + (e0 >> 3);
    if constexpr (kWords == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      word[0] = v.x; word[1] = v.y;
    } else {
#pragma unroll
      for (int q = 0; q < kWords / 4; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(p)[q];
        word[4 * q] = v.x; word[4 * q + 1] = v.y; word[4 * q + 2] = v.z; word[4 * q + 3] = v.w;
      }
    }
#pragma unroll
    for (int r = 0; r < kRuns; ++r) sc[r] = load_scale(w, nested, e0 + 32 * r);
  }
  __device__ __forceinline__ void store(uint4* tile, const float* s_code, const float* s_code2,
                                        float off, int nested) const {
    using L = LdsRows<kBK>;
    float s[kRuns];
#pragma unroll
    for (int r = 0; r < kRuns; ++r)
      s[r] = block_scale(nested, s_code2[nested ? sc[r].q8 : 0], sc[r].a2, off, sc[r].a2);
#pragma unroll
    for (int q = 0; q < kWords; ++q) {
      const float sq = s[(q * 8) / 32 < kRuns ? (q * 8) / 32 : kRuns - 1];
      uint32_t h[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (word[q] >> (8 * b)) & 0xffu;
        h[b] = pack2(s_code[byte >> 4] * sq, s_code[byte & 0xfu] * sq);
      }
      const int lc = part * kWords + q;
      tile[row * L::kRC + (lc ^ L::swz(row))] = make_uint4(h[0], h[1], h[2], h[3]);
    }
  }
};

// Backward: tile rows = weight columns k0 .. k0 + BM, contraction = weight rows n0 .. n0 + 64.
// A lane takes RPT = BM / 32 consecutive weight rows x 8 consecutive columns (one 4-byte word
// per row, one block scale per row) and writes, for each of its 8 columns, RPT values into one
// piece of an LDS chunk.
template <int BM>
struct BwdLoader {
  static constexpr int kRPT = BM / 32;     // weight rows per lane
  static constexpr int kNG = kBK / kRPT;   // lanes along the contraction
  static_assert(kRPT == 2 || kRPT == 4 || kRPT == 8, "BM of 64, 128 or 256");
  uint32_t word[kRPT];
  ScaleRaw sc[kRPT];
  int kw, ng;

  __device__ __forceinline__ void init(int tid) {
    ng = tid % kNG;
    kw = tid / kNG;
  }
  __device__ __forceinline__ void load(const WeightDev& w, int nested, int cols, int n0, int k0) {
#pragma unroll
    for (int r = 0; r < kRPT; ++r) {
      const int64_t e0 = static_cast<int64_t>(n0 + ng * kRPT + r) * cols + k0 + kw * 8;
      word[r] = w.packed[e0 >> 3];
      sc[r] = load_scale(w, nested, e0);
    }
  }
  __device__ __forceinline__ void store(uint4* tile, const float* s_code, const float* s_code2,
                                        float off, int nested) const {
    using L = LdsRows<kBK>;
    float s[kRPT];
#pragma unroll
    for (int r = 0; r < kRPT; ++r)
      s[r] = block_scale(nested, s_code2[nested ? sc[r].q8 : 0], sc[r].a2, off, sc[r].a2);
    const int ncol = ng * kRPT;  // first contraction column of the lane's piece
    const int lc = ncol / 8;
    char* base = reinterpret_cast<char*>(tile);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // element j of each row's word: byte j / 2, high nibble for even j
      float v[kRPT];
#pragma unroll
      for (int r = 0; r < kRPT; ++r) {
        const uint32_t byte = (word[r] >> (8 * (j / 2))) & 0xffu;
        const uint32_t nib = (j % 2 == 0) ? (byte >> 4) : (byte & 0xfu);
        v[r] = s_code[nib] * s[r];
      }
      const int kk = kw * 8 + j;
      char* dst = base + (kk * L::kRC + (lc ^ L::swz(kk))) * 16 + (ncol % 8) * 2;
      if constexpr (kRPT == 8) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]),
                                                    pack2(v[4], v[5]), pack2(v[6], v[7]));
      } else if constexpr (kRPT == 4) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
      } else {
        *reinterpret_cast<uint32_t*>(dst) = pack2(v[0], v[1]);
      }
    }
  }
};

// ---------------------------------------------------------------------------------------------
template <int BM, int BN, bool TRANS>
__global__ __launch_bounds__(kThreads, 2) void nf4_gemm_kernel(const Args args) {
  using L = LdsRows<kBK>;
  constexpr int kRC = L::kRC;
  constexpr int kStage = (BM + BN) * kRC;  // uint4 per stage
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  using TB = DmaTile<BN, 4, kBK>;
  using Loader = typename std::conditional<TRANS, BwdLoader<BM>, FwdLoader<BM>>::type;

  __shared__ uint4 ring[2 * kStage];
  __shared__ float s_code[kMaxW][16];
  __shared__ float s_code2[kMaxW][256];
  __shared__ float s_off[kMaxW];

  const int tid = threadIdx.x;
  const int lane = tid % cm::kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / cm::kWave);
  const int wm = wave / 2, wn = wave % 2;
  const int nested = args.nested;

  for (int i = 0; i < args.n_w; ++i) {
    if (tid < 16) s_code[i][tid] = args.w[i].code[tid];
    if (nested) {
      s_code2[i][tid] = args.w[i].code2[tid];
      if (tid == 0) s_off[i] = *args.w[i].offset;
    } else if (tid == 0) {
      s_off[i] = 0.0f;
    }
  }

  // tile of this workgroup: a (weight side) and b (tokens), consecutive ids share the a tile
  int bid = blockIdx.x;
  if (args.remap) {
    const int per = gridDim.x / 8;
    bid = (bid % 8) * per + bid / 8;
  }
  const int ta = bid / args.tiles_b, tb = bid % args.tiles_b;
  const int m0 = tb * BN;

  // forward: the weight holding tile ta, its first row; backward: the weight columns
  int wf = 0;
  if constexpr (!TRANS) {
    while (wf + 1 < args.n_w && ta >= args.w[wf + 1].first) ++wf;
  }
  const int a0 = TRANS ? ta * BM : (ta - args.w[wf].first) * BM;
  const int n_kt = TRANS ? args.n_stages : args.cols / kBK;

  // stage kt -> weight index and contraction offset within it
  auto stage_w = [&](int kt) {
    if constexpr (!TRANS) {
      return wf;
    } else {
      int i = 0;
      while (i + 1 < args.n_w && kt >= args.w[i + 1].first) ++i;
      return i;
    }
  };
  auto stage_k = [&](int kt, int wi) { return TRANS ? (kt - args.w[wi].first) * kBK : kt * kBK; };
  auto token_src = [&](int wi) {
    RowMajor s;
    if constexpr (TRANS) {
      s.p = args.w[wi].g;
      s.ld = args.w[wi].ldg;
      s.k_len = args.w[wi].rows;
    } else {
      s.p = args.x;
      s.ld = args.ldx;
      s.k_len = args.cols;
    }
    s.rows = args.m;
    return s;
  };

  Loader ld;
  ld.init(tid);
  TB lb;
  auto load_a = [&](int kt) {
    const int wi = stage_w(kt), kc = stage_k(kt, wi);
    if constexpr (TRANS) {
      ld.load(args.w[wi], nested, args.cols, kc, a0);
    } else {
      ld.load(args.w[wi], nested, args.cols, a0, kc);
    }
  };
  auto store_a = [&](int kt, uint4* st) {
    const int wi = stage_w(kt);
    ld.store(st, s_code[wi], s_code2[wi], s_off[wi], nested);
  };
  auto issue_b = [&](int kt, uint4* st) {
    const int wi = stage_w(kt), kc = stage_k(kt, wi);
    const RowMajor src = token_src(wi);
    lb.init(src, wave, lane);
    const bool inside = src.tile_inside(m0, BN, kc);
#pragma unroll
    for (int q = 0; q < TB::kPer; ++q) lb.issue(src, m0, kc, st + BM * kRC, wave, q, inside);
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // prologue: stage 0 in buffer 0, the packed bytes of stage 1 in registers
  load_a(0);
  issue_b(0, ring);
  __syncthreads();  // the code tables
  store_a(0, ring);
  cm::gemm::wait_vmcnt<0>();  // the token tile of stage 0
  if (n_kt > 1) load_a(1);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  cm::gemm::lds_barrier();

  const int arow = wm * WTM + lane % 32, brow = wn * WTN + lane % 32;
  for (int kt = 0; kt < n_kt; ++kt) {
    uint4* cur = ring + (kt & 1) * kStage;
    uint4* nxt = ring + ((kt + 1) & 1) * kStage;
    const bool more = kt + 1 < n_kt;
    if (more) issue_b(kt + 1, nxt);
    const uint4* As = cur;
    const uint4* Bs = cur + BM * kRC;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int ch = ks * 2 + lane / 32;
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = L::frag(As, arow + i * 32, ch);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = L::frag(Bs, brow + j * 32, ch);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_a(kt + 1, nxt);
    // the token tile of stage kt + 1 has landed; the packed bytes of stage kt + 2 are loaded
    // after this wait and stay in flight through the barrier and the next stage's products
    cm::gemm::wait_vmcnt<0>();
    if (kt + 2 < n_kt) load_a(kt + 2);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this lane's LDS writes have landed
    cm::gemm::lds_barrier();
  }

  // epilogue: lane holds C[a][t] for tokens t = m0 + wn * WTN + j * 32 + lane % 32 and weight-side
  // rows a = a0 + wm * WTM + i * 32 + (e / 4) * 8 + (lane / 32) * 4 + e % 4: 4 consecutive
  // outputs of one token row per (i, j, e / 4)
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int t = m0 + wn * WTN + j * 32 + lane % 32;
    if (t >= args.m) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int a = a0 + wm * WTM + i * 32 + g * 8 + (lane / 32) * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][g * 4 + e];
        void* out;
        int64_t off;
        if constexpr (TRANS) {
          out = args.dx;
          off = static_cast<int64_t>(t) * args.lddx + a;
        } else {
          const WeightDev& w = args.w[wf];
          if (w.bias) {
            const uint2 bb = *reinterpret_cast<const uint2*>(w.bias + a);
            const _Float16* bh = reinterpret_cast<const _Float16*>(&bb);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += static_cast<float>(bh[e]);
          }
          out = w.out;
          off = static_cast<int64_t>(t) * w.ldo + a;
        }
        if (args.out32) {
          float4 o;
          o.x = cm::round_to<_Float16>(v[0]);
          o.y = cm::round_to<_Float16>(v[1]);
          o.z = cm::round_to<_Float16>(v[2]);
          o.w = cm::round_to<_Float16>(v[3]);
          *reinterpret_cast<float4*>(static_cast<float*>(out) + off) = o;
        } else {
          *reinterpret_cast<uint2*>(static_cast<_Float16*>(out) + off) =
              make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Wavefront-specialized version for weights with a scale map (fp32 block scales decoded once per
// weight, cm_nf4_scale_map), tiles of BM = 128 or 256 weight-side rows x 128 tokens, one
// workgroup of 8 wavefronts per CU.
//
// Wavefronts 0-3 (consumers, a 2 x 2 grid) only read LDS fragments and issue MFMAs. Wavefronts
// 4-7 (producers) move every byte from HBM/L2 by direct-to-LDS loads (global_load_lds), so the
// only memory waits in the loop are the producers' explicit vmcnt waits:
//   - raw stage data in a ring of 3 slots, issued two stages ahead: the token tile (read by the
//     consumers), and the packed weight bytes and block scales, each into the slot of the lane
//     that expands them (lane-private, so a lane's own vmcnt wait makes them visible to it);
//   - the expanded fp16 weight tile in a double buffer, written one stage ahead.
// Per stage kt a producer lane issues the raw loads of stage kt + 2, waits for those of stage
// kt + 1 and expands stage kt + 1; the consumers multiply stage kt. One barrier per stage.
//
// Expansion, forward: a lane owns EPT = BM / 4 consecutive elements of one weight row, all in one
// block (blocksize >= 64), so it builds the block's 16 products fp16(code[i] * s) once and maps
// nibbles to them with byte permutes (v_perm_b32 over the products' low- and high-byte planes):
// no per-element multiply and no LDS lookups. Backward: a lane owns RPT = BM / 32 weight rows x
// 8 columns, one scale per row; each value is fp16(code[nibble] * s_row) with the 16-entry code
// table in LDS. Both give exactly the dequant kernel's fp16 values.
//
// The contraction may be split over gridDim: slice s of S covers stages [s n / S, (s + 1) n / S)
// and writes fp32 partial sums; nf4_gemm_reduce adds the slices in order (deterministic), adds
// the bias and rounds.
constexpr int kConsumers = 8;  // MFMA wavefronts: 4 x 2 (256-row tiles) or 2 x 4 (128-row)
constexpr int kProducers = 4;
constexpr int kWsThreads = (kConsumers + kProducers) * 64;
constexpr int kRing = 3;
constexpr int kWsBN = 128;

// One global_load_lds_dword: lane l's 4 bytes from g land at lds_lane0 + 4 l (wave-uniform base in
// M0); issued like gemm::dma16.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma4(const void* g, void* lds_lane0) {
  const uint32_t m0v = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((cm::gemm::lds_ptr_t)lds_lane0));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(m0v), "v"(g)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// The 16 products fp16(code[i] * s) as byte planes: lo[q] holds the low bytes of products
// 4q .. 4q + 3, hi[q] their high bytes.
struct ProductPlanes {
  uint32_t lo[4], hi[4];
  __device__ __forceinline__ void build(const float (&code)[16], float s) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t d0 = pack2(code[4 * q] * s, code[4 * q + 1] * s);
      const uint32_t d1 = pack2(code[4 * q + 2] * s, code[4 * q + 3] * s);
      lo[q] = __builtin_amdgcn_perm(d1, d0, 0x06040200u);
      hi[q] = __builtin_amdgcn_perm(d1, d0, 0x07050301u);
    }
  }
  // x: four nibble values, one per byte -> (low bytes, high bytes) of their products
  __device__ __forceinline__ void lookup(uint32_t x, uint32_t& l, uint32_t& h) const {
    const uint32_t sel = x & 0x07070707u;
    // 0xff in the bytes whose nibble is >= 8 (selector 0x0d gives 0xff, 0x0c gives 0x00)
    const uint32_t msk = __builtin_amdgcn_perm(0u, 0u, ((x >> 3) & 0x01010101u) | 0x0c0c0c0cu);
    const uint32_t l0 = __builtin_amdgcn_perm(lo[1], lo[0], sel);
    const uint32_t l1 = __builtin_amdgcn_perm(lo[3], lo[2], sel);
    const uint32_t h0 = __builtin_amdgcn_perm(hi[1], hi[0], sel);
    const uint32_t h1 = __builtin_amdgcn_perm(hi[3], hi[2], sel);
    l = (l1 & msk) | (l0 & ~msk);
    h = (h1 & msk) | (h0 & ~msk);
  }
  // one packed word (elements 2b in the high nibble, 2b + 1 in the low nibble of byte b) ->
  // its 8 fp16 values in element order, as 4 dwords
  __device__ __forceinline__ uint4 expand(uint32_t w) const {
    uint32_t le, he, lo_, ho;
    lookup((w >> 4) & 0x0f0f0f0fu, le, he);  // elements 0, 2, 4, 6
    lookup(w & 0x0f0f0f0fu, lo_, ho);        // elements 1, 3, 5, 7
    const uint32_t e02 = __builtin_amdgcn_perm(he, le, 0x05010400u);  // e0 | e2 << 16
    const uint32_t e46 = __builtin_amdgcn_perm(he, le, 0x07030602u);
    const uint32_t o13 = __builtin_amdgcn_perm(ho, lo_, 0x05010400u);  // e1 | e3 << 16
    const uint32_t o57 = __builtin_amdgcn_perm(ho, lo_, 0x07030602u);
    return make_uint4(__builtin_amdgcn_perm(o13, e02, 0x05040100u),   // e0 | e1 << 16
                      __builtin_amdgcn_perm(o13, e02, 0x07060302u),   // e2 | e3 << 16
                      __builtin_amdgcn_perm(o57, e46, 0x05040100u),
                      __builtin_amdgcn_perm(o57, e46, 0x07060302u));
  }
};

template <int BM, int BN, bool TRANS>
struct V3Layout {
  static constexpr int kEPT = BM / 4;                 // forward: elements per lane
  static constexpr int kTPR = kBK / kEPT;             // forward: lanes per weight row
  static constexpr int kRPT = BM / 32;                // backward: weight rows per lane
  static constexpr int kNG = kBK / kRPT;              // backward: lanes along the contraction
  static constexpr int kA16 = BM * 8;                 // uint4 of an expanded weight tile
  static constexpr int kBt = BN * 8;                  // uint4 of a token tile
  static constexpr int kPk = TRANS ? kRPT * 64 : (kEPT / 32) * 256;  // uint4 of packed bytes
  static constexpr int kSc = 64;                      // uint4 of block scales (1 KB)
  static constexpr int kSlot = kBt + kPk + kSc;
  // direct-to-LDS instructions a producer lane issues per stage
  static constexpr int kIssue = BN / 32 + (TRANS ? kRPT : kEPT / 32) + 1;
};

template <int BM, int BN, bool TRANS>
__global__ __launch_bounds__(kWsThreads, 1) void nf4_gemm_v3(const Args args) {
  using L = LdsRows<kBK>;
  using Y = V3Layout<BM, BN, TRANS>;
  constexpr int kRC = L::kRC;
  constexpr int WN = BN / 64, WM = kConsumers / WN;  // 64 x 64 wavefront tiles
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int KS = kBK / 16;
  using TB = DmaTile<BN, kProducers, kBK>;

  __shared__ uint4 a16[2 * Y::kA16];
  __shared__ uint4 raw[kRing * Y::kSlot];
  __shared__ float s_code[kMaxW][16];

  const int tid = threadIdx.x;
  const int lane = tid % cm::kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / cm::kWave);
  const bool producer = wave >= kConsumers;
  const int p = tid - kConsumers * cm::kWave;  // producer lane 0..255

  if (producer) {
    for (int i = 0; i < args.n_w; ++i)
      if (p < 16) s_code[i][p] = args.w[i].code[p];
  }

  int bid = blockIdx.x;
  if (args.remap) {
    const int per = gridDim.x / 8;
    bid = (bid % 8) * per + bid / 8;
  }
  const int n_tiles = gridDim.x / args.split;
  const int slice = bid / n_tiles;
  const int tile = bid % n_tiles;
  const int ta = tile / args.tiles_b, tb = tile % args.tiles_b;
  const int m0 = tb * BN;
  int wf = 0;
  if constexpr (!TRANS) {
    while (wf + 1 < args.n_w && ta >= args.w[wf + 1].first) ++wf;
  }
  const int a0 = TRANS ? ta * BM : (ta - args.w[wf].first) * BM;
  const int n_all = TRANS ? args.n_stages : args.cols / kBK;
  const int kb = static_cast<int>(static_cast<int64_t>(slice) * n_all / args.split);
  const int ke = static_cast<int>(static_cast<int64_t>(slice + 1) * n_all / args.split);
  const int n_loc = ke - kb;
  const int cols = args.cols;

  __syncthreads();  // the code tables

  if (producer) {
    const int pw = wave - kConsumers;
    TB lb;
    float code[16];
    if constexpr (!TRANS) {
#pragma unroll
      for (int i = 0; i < 16; ++i) code[i] = s_code[wf][i];
    }
    // forward lane: weight row a0 + row, elements part * EPT .. + EPT of the stage
    const int row = p / Y::kTPR, part = p % Y::kTPR;
    // backward lane: weight rows ng * RPT .. + RPT of the stage, columns a0 + kw * 8 .. + 8
    const int ng = p % Y::kNG, kw = p / Y::kNG;
    auto stage_w = [&](int kt) {
      int i = 0;
      if constexpr (TRANS) {
        while (i + 1 < args.n_w && kt >= args.w[i + 1].first) ++i;
      } else {
        i = wf;
      }
      return i;
    };
    auto issue = [&](int kt, uint4* slot) {
      const int wi = stage_w(kt);
      const WeightDev& w = args.w[wi];
      const int kc = TRANS ? (kt - w.first) * kBK : kt * kBK;
      RowMajor src;
      if constexpr (TRANS) {
        src.p = w.g;
        src.ld = w.ldg;
        src.k_len = w.rows;
      } else {
        src.p = args.x;
        src.ld = args.ldx;
        src.k_len = cols;
      }
      src.rows = args.m;
      lb.init(src, pw, lane);
      const bool inside = src.tile_inside(m0, BN, kc);
#pragma unroll
      for (int q = 0; q < TB::kPer; ++q) lb.issue(src, m0, kc, slot, pw, q, inside);
      const char* pk = reinterpret_cast<const char*>(w.packed);
      uint4* pk_lds = slot + Y::kBt;
      uint4* sc_lds = pk_lds + Y::kPk;
      if constexpr (!TRANS) {
        const int64_t e0 = static_cast<int64_t>(a0 + row) * cols + kc + part * Y::kEPT;
#pragma unroll
        for (int i = 0; i < Y::kEPT / 32; ++i)
          cm::gemm::dma16(pk + e0 / 2 + 16 * i, pk_lds + i * 256 + pw * 64);
        const int64_t cb = (kc + part * Y::kEPT) >> w.bs_shift;
        dma4(w.smap + cb * w.rows + a0 + row, reinterpret_cast<float*>(sc_lds) + pw * 64);
      } else {
#pragma unroll
        for (int r = 0; r < Y::kRPT; ++r) {
          const int64_t e0 = static_cast<int64_t>(kc + ng * Y::kRPT + r) * cols + a0 + kw * 8;
          dma4(pk + e0 / 2, reinterpret_cast<uint32_t*>(pk_lds) + r * 256 + pw * 64);
        }
        // the wave's 64 weight columns lie in one block: its scales of the stage's 64 rows
        const int64_t cb = static_cast<int64_t>(a0 + pw * (BM / 4)) >> w.bs_shift;
        if (lane < 16) cm::gemm::dma16(w.smap + cb * w.rows + kc + lane * 4, sc_lds + pw * 16);
      }
    };
    auto expand = [&](int kt, const uint4* slot, uint4* dst) {
      const uint4* pk_lds = slot + Y::kBt;
      const uint4* sc_lds = pk_lds + Y::kPk;
      if constexpr (!TRANS) {
        const float s = reinterpret_cast<const float*>(sc_lds)[p];
        ProductPlanes pl;
        pl.build(code, s);
#pragma unroll
        for (int i = 0; i < Y::kEPT / 32; ++i) {
          const uint4 v = pk_lds[i * 256 + p];
          const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int lc = part * (Y::kEPT / 8) + i * 4 + q;
            dst[row * kRC + (lc ^ L::swz(row))] = pl.expand(wd[q]);
          }
        }
      } else {
        const int wi = stage_w(kt);
        const float* cd = s_code[wi];
        const uint32_t* pk32 = reinterpret_cast<const uint32_t*>(pk_lds);
        const float* scf = reinterpret_cast<const float*>(sc_lds) + pw * 64 + ng * Y::kRPT;
        uint32_t wd[Y::kRPT];
        float s[Y::kRPT];
#pragma unroll
        for (int r = 0; r < Y::kRPT; ++r) {
          wd[r] = pk32[r * 256 + p];
          s[r] = scf[r];
        }
        const int ncol = ng * Y::kRPT;
        char* base = reinterpret_cast<char*>(dst);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float v[Y::kRPT];
#pragma unroll
          for (int r = 0; r < Y::kRPT; ++r) {
            const uint32_t byte = (wd[r] >> (8 * (j / 2))) & 0xffu;
            v[r] = cd[(j % 2 == 0) ? (byte >> 4) : (byte & 0xfu)] * s[r];
          }
          const int kk = kw * 8 + j;
          char* d = base + (kk * kRC + ((ncol / 8) ^ L::swz(kk))) * 16 + (ncol % 8) * 2;
          if constexpr (Y::kRPT == 8) {
            *reinterpret_cast<uint4*>(d) = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]),
                                                      pack2(v[4], v[5]), pack2(v[6], v[7]));
          } else {
            *reinterpret_cast<uint2*>(d) = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
          }
        }
      }
    };
    // prologue: raw stages 0 and 1 in flight, stage 0 expanded
    issue(kb, raw);
    if (1 < n_loc) {
      issue(kb + 1, raw + Y::kSlot);
      cm::gemm::wait_vmcnt<Y::kIssue>();
    } else {
      cm::gemm::wait_vmcnt<0>();
    }
    expand(kb, raw, a16);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    cm::gemm::lds_barrier();
    for (int kt = 0; kt < n_loc; ++kt) {
      if (kt + 2 < n_loc) {
        issue(kb + kt + 2, raw + ((kt + 2) % kRing) * Y::kSlot);
        cm::gemm::wait_vmcnt<Y::kIssue>();  // the raw data of stage kt + 1 has landed
      } else {
        cm::gemm::wait_vmcnt<0>();
      }
      if (kt + 1 < n_loc)
        expand(kb + kt + 1, raw + ((kt + 1) % kRing) * Y::kSlot, a16 + ((kt + 1) & 1) * Y::kA16);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // this lane's LDS writes have landed
      cm::gemm::lds_barrier();
    }
    return;
  }

  // consumers
  const int wm = wave / WN, wn = wave % WN;
  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  cm::gemm::lds_barrier();  // stage 0 is in place
  const int arow = wm * WTM + lane % 32, brow = wn * WTN + lane % 32;
  for (int kt = 0; kt < n_loc; ++kt) {
    const uint4* As = a16 + (kt & 1) * Y::kA16;
    const uint4* Bs = raw + (kt % kRing) * Y::kSlot;
    half8 af[2][TM], bf[2][TN];
    auto read = [&](int ks, int b) {
      const int ch = ks * 2 + lane / 32;
#pragma unroll
      for (int i = 0; i < TM; ++i) af[b][i] = L::frag(As, arow + i * 32, ch);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[b][j] = L::frag(Bs, brow + j * 32, ch);
    };
    read(0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read(ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks & 1][i], bf[ks & 1][j],
                                                             acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    cm::gemm::lds_barrier();
  }

  // epilogue: lane holds C[a][t] for tokens t = m0 + wn * WTN + j * 32 + lane % 32 and weight-side
  // rows a = a0 + wm * WTM + i * 32 + (e / 4) * 8 + (lane / 32) * 4 + e % 4; a split writes fp32
  // partials of its slice
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int t = m0 + wn * WTN + j * 32 + lane % 32;
    if (t >= args.m) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int a = a0 + wm * WTM + i * 32 + g * 8 + (lane / 32) * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][g * 4 + e];
        if (args.split > 1) {
          float* dst = args.ws + (static_cast<int64_t>(slice) * args.m + t) * args.n_out + a;
          *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
          continue;
        }
        void* out;
        int64_t off;
        if constexpr (TRANS) {
          out = args.dx;
          off = static_cast<int64_t>(t) * args.lddx + a;
        } else {
          const WeightDev& w = args.w[wf];
          if (w.bias) {
            const uint2 bb = *reinterpret_cast<const uint2*>(w.bias + a);
            const _Float16* bh = reinterpret_cast<const _Float16*>(&bb);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += static_cast<float>(bh[e]);
          }
          out = w.out;
          off = static_cast<int64_t>(t) * w.ldo + a;
        }
        if (args.out32) {
          *reinterpret_cast<float4*>(static_cast<float*>(out) + off) =
              make_float4(cm::round_to<_Float16>(v[0]), cm::round_to<_Float16>(v[1]),
                          cm::round_to<_Float16>(v[2]), cm::round_to<_Float16>(v[3]));
        } else {
          *reinterpret_cast<uint2*>(static_cast<_Float16*>(out) + off) =
              make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
        }
      }
    }
  }
}

// Block scales as an fp32 map, transposed: smap[c][r] = the scale of the block that holds
// element (r, c * blocksize) (cols a multiple of the blocksize, so a block never crosses rows).
__global__ __launch_bounds__(256) void nf4_scale_map_kernel(WeightDev w, int nested, int cols,
                                                             float* __restrict__ smap) {
  const int64_t nb_row = cols >> w.bs_shift;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // = c * rows + r
  if (i >= nb_row * w.rows) return;
  const int64_t c = i / w.rows, r = i % w.rows;
  const int64_t blk = r * nb_row + c;
  const ScaleRaw raw = load_scale(w, nested, blk << w.bs_shift);
  smap[i] = nested ? block_scale(1, w.code2[raw.q8], raw.a2, *w.offset, 0.0f) : raw.a2;
}

// Sum of the split's fp32 partials in slice order, plus the bias, rounded to fp16 (and widened
// with out32). One lane per 4 consecutive outputs.
__global__ __launch_bounds__(256) void nf4_gemm_reduce(const float* __restrict__ ws, int split,
                                                        int m, int n_out,
                                                        const _Float16* __restrict__ bias,
                                                        void* out, int64_t ldo, int out32) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int quads = n_out / 4;
  if (q >= static_cast<int64_t>(m) * quads) return;
  const int t = static_cast<int>(q / quads), a = static_cast<int>(q % quads) * 4;
  const int64_t slice_stride = static_cast<int64_t>(m) * n_out;
  const float* src = ws + static_cast<int64_t>(t) * n_out + a;
  float4 acc = *reinterpret_cast<const float4*>(src);
  for (int s = 1; s < split; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(src + s * slice_stride);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  if (bias) {
    acc.x += static_cast<float>(bias[a]);
    acc.y += static_cast<float>(bias[a + 1]);
    acc.z += static_cast<float>(bias[a + 2]);
    acc.w += static_cast<float>(bias[a + 3]);
  }
  const int64_t off = static_cast<int64_t>(t) * ldo + a;
  if (out32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + off) =
        make_float4(cm::round_to<_Float16>(acc.x), cm::round_to<_Float16>(acc.y),
                    cm::round_to<_Float16>(acc.z), cm::round_to<_Float16>(acc.w));
  } else {
    *reinterpret_cast<uint2*>(static_cast<_Float16*>(out) + off) =
        make_uint2(pack2(acc.x, acc.y), pack2(acc.z, acc.w));
  }
}

// ---------------------------------------------------------------------------------------------
int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

constexpr int kCUs = 256;

template <int BM, int BN, bool TRANS>
int launch_cfg(const Args& a, int n_tiles, hipStream_t stream) {
  hipLaunchKernelGGL((nf4_gemm_kernel<BM, BN, TRANS>), dim3(static_cast<uint32_t>(n_tiles)),
                     dim3(kThreads), 0, stream, a);
  return cm::launch_status();
}

// Common checks and device views of the weights; 0 or an error code.
int setup(const cm_nf4_weight* w, int n_w, int64_t m, Args& a) {
  CM_CHECK_ARG(w != nullptr && n_w >= 1 && n_w <= kMaxW);
  CM_CHECK_ARG(m >= 0 && m < (int64_t{1} << 31));
  const int64_t cols = w[0].cols;
  CM_CHECK_ARG(cols > 0 && cols % kBK == 0 && cols < (int64_t{1} << 30));
  a = Args{};
  a.n_w = n_w;
  a.nested = w[0].nested ? 1 : 0;
  a.cols = static_cast<int>(cols);
  a.m = static_cast<int>(m);
  for (int i = 0; i < n_w; ++i) {
    const cm_nf4_weight& s = w[i];
    CM_CHECK_ARG(s.packed && s.absmax && s.code);
    CM_CHECK_ARG(s.cols == cols && s.rows > 0 && s.rows % kBK == 0 &&
                 s.rows < (int64_t{1} << 30));
    // 32-bit block indices; 4-byte aligned packed rows (cols a multiple of 64)
    CM_CHECK_ARG(s.rows * cols / 32 < (int64_t{1} << 31));
    CM_CHECK_ARG(cm::aligned(s.packed, 16));
    CM_CHECK_ARG((s.nested ? 1 : 0) == a.nested);
    const int bs_shift = log2_exact(s.blocksize);
    CM_CHECK_ARG(bs_shift >= 5);  // blocksize >= 32, a power of two
    if (a.nested) CM_CHECK_ARG(s.code2 && s.absmax2 && s.offset && s.blocksize2 >= 1);
    WeightDev& d = a.w[i];
    d.packed = reinterpret_cast<const uint32_t*>(s.packed);
    d.smap = s.scale_map;
    if (d.smap) CM_CHECK_ARG(cm::aligned(d.smap, 16));
    d.absmax = s.absmax;
    d.absmax2 = s.absmax2;
    d.offset = s.offset;
    d.code = s.code;
    d.code2 = s.code2;
    d.rows = static_cast<int>(s.rows);
    d.bs_shift = bs_shift;
    d.bs2_shift = a.nested ? log2_exact(s.blocksize2) : 0;
    d.bs2 = a.nested ? static_cast<uint32_t>(s.blocksize2) : 1u;
  }
  return 0;
}

// Tile shape per call for the general kernel: the largest tiles that still give every CU a
// workgroup; the smallest when none does.
template <class TilesFn>
void pick_tiles(TilesFn tiles, bool allow128, int& bm, int& bn) {
  const int cand[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
  for (const auto& c : cand) {
    if (c[0] == 128 && !allow128) continue;
    if (tiles(c[0], c[1]) >= kCUs) {
      bm = c[0];
      bn = c[1];
      return;
    }
  }
  bm = 64;
  bn = 64;
}

// How one call runs: the wavefront-specialized kernel (ws) when the weights have scale maps and
// the weight-side extent is a multiple of 128, with the contraction split when the tiles alone
// leave CUs idle; the general kernel otherwise.
struct Plan {
  bool ws;
  int bm, bn, split;
  int64_t tiles;     // output tiles (workgroups = tiles * split)
  int n_out;         // output columns (weight rows forward, weight columns backward)
  int64_t ws_bytes;  // fp32 partials of a split
};

Plan plan_for(const Args& a, bool trans) {
  Plan p{};
  const int64_t tb = (static_cast<int64_t>(a.m) + kWsBN - 1) / kWsBN;
  int64_t rows_total = 0;
  bool all128 = true, all256 = true;
  for (int i = 0; i < a.n_w; ++i) {
    rows_total += a.w[i].rows;
    all128 = all128 && a.w[i].rows % 128 == 0;
    all256 = all256 && a.w[i].rows % 256 == 0;
  }
  const int extent = trans ? a.cols : static_cast<int>(rows_total);
  bool maps = true;  // every weight has a scale map with blocks of >= 64 that never cross rows
  for (int i = 0; i < a.n_w; ++i)
    maps = maps && a.w[i].smap && a.w[i].bs_shift >= 6 && (a.cols >> a.w[i].bs_shift) > 0 &&
           a.cols % (1 << a.w[i].bs_shift) == 0;
  const bool e128 = maps && (trans ? a.cols % 128 == 0 : all128);
  const bool e256 = trans ? a.cols % 256 == 0 : all256;
  p.n_out = trans ? a.cols : (a.n_w == 1 ? a.w[0].rows : 0);
  if (e128) {
    p.ws = true;
    p.bn = kWsBN;
    p.bm = e256 ? 256 : 128;
    p.tiles = extent / p.bm * tb;
    if (p.bm == 256 && p.tiles < kCUs / 2) {
      p.bm = 128;
      p.tiles = extent / p.bm * tb;
    }
    // 256-token tiles expand each weight element half as often; taken when they, split over the
    // contraction where that is allowed, still give most CUs a workgroup
    const int64_t tb2 = (static_cast<int64_t>(a.m) + 255) / 256;
    const int64_t tiles2 = extent / 128 * tb2;
    const bool can_split = trans || a.n_w == 1;
    const int n_stages_all = trans ? a.n_stages : a.cols / kBK;
    int64_t sp2 = 1;
    if (can_split && tiles2 < kCUs * 3 / 4) {
      sp2 = kCUs / (tiles2 > 0 ? tiles2 : 1);
      if (sp2 > 8) sp2 = 8;
      if (sp2 > n_stages_all / 8) sp2 = n_stages_all / 8;
      if (sp2 < 1) sp2 = 1;
    }
    if (a.m >= 384 && tiles2 * sp2 >= kCUs * 3 / 4) {
      p.bm = 128;
      p.bn = 256;
      p.tiles = tiles2;
    }
    const int n_all = trans ? a.n_stages : a.cols / kBK;
    p.split = 1;
    if (p.tiles < 3 * kCUs / 4 && (trans || a.n_w == 1)) {
      int64_t sp = kCUs / (p.tiles > 0 ? p.tiles : 1);
      if (sp > 8) sp = 8;
      if (sp > n_all / 8) sp = n_all / 8;
      if (sp > 1) p.split = static_cast<int>(sp);
    }
    p.ws_bytes = p.split > 1 ? int64_t{4} * p.split * a.m * p.n_out : 0;
    return p;
  }
  p.ws = false;
  p.split = 1;
  auto tiles = [&](int bm, int bn) {
    return static_cast<int64_t>(extent / bm) * ((a.m + bn - 1) / bn);
  };
  pick_tiles(tiles, trans ? a.cols % 128 == 0 : all128, p.bm, p.bn);
  p.tiles = tiles(p.bm, p.bn);
  return p;
}

template <int BM, int BN, bool TRANS>
int launch_ws(const Args& a, int64_t blocks, hipStream_t stream) {
  hipLaunchKernelGGL((nf4_gemm_v3<BM, BN, TRANS>), dim3(static_cast<uint32_t>(blocks)),
                     dim3(kWsThreads), 0, stream, a);
  return cm::launch_status();
}

// Launch per plan (first fields of `first` already set: the forward's tile offsets are filled
// here). out/ldo/bias of the reduce: the one output of the call.
int run(Args& a, Plan p, bool trans, void* workspace, int64_t ws_bytes, void* out, int64_t ldo,
        const _Float16* bias, hipStream_t s) {
  if (p.ws && p.split > 1 &&
      (workspace == nullptr || ws_bytes < p.ws_bytes || !cm::aligned(workspace, 16))) {
    p.split = 1;  // no room for the partials: one slice (same results, fewer workgroups)
  }
  if (!trans) {
    int first = 0;
    for (int i = 0; i < a.n_w; ++i) {
      a.w[i].first = first;
      first += a.w[i].rows / p.bm;
    }
  }
  a.tiles_b = static_cast<int>((a.m + p.bn - 1) / p.bn);
  const int64_t blocks = p.tiles * p.split;
  CM_CHECK_ARG(blocks > 0 && blocks < 0x7fffffff);
  a.remap = blocks % 8 == 0;
  a.split = p.split;
  a.ws = p.split > 1 ? static_cast<float*>(workspace) : nullptr;
  a.n_out = p.n_out;
  int st;
  if (p.ws) {
    if (p.bn == 256) {
      st = trans ? launch_ws<128, 256, true>(a, blocks, s) : launch_ws<128, 256, false>(a, blocks, s);
    } else if (trans) {
      st = p.bm == 256 ? launch_ws<256, 128, true>(a, blocks, s)
                       : launch_ws<128, 128, true>(a, blocks, s);
    } else {
      st = p.bm == 256 ? launch_ws<256, 128, false>(a, blocks, s)
                       : launch_ws<128, 128, false>(a, blocks, s);
    }
  } else {
    const int nt = static_cast<int>(blocks);
    if (trans) {
      if (p.bm == 128 && p.bn == 128) st = launch_cfg<128, 128, true>(a, nt, s);
      else if (p.bm == 128) st = launch_cfg<128, 64, true>(a, nt, s);
      else if (p.bn == 128) st = launch_cfg<64, 128, true>(a, nt, s);
      else st = launch_cfg<64, 64, true>(a, nt, s);
    } else {
      if (p.bm == 128 && p.bn == 128) st = launch_cfg<128, 128, false>(a, nt, s);
      else if (p.bm == 128) st = launch_cfg<128, 64, false>(a, nt, s);
      else if (p.bn == 128) st = launch_cfg<64, 128, false>(a, nt, s);
      else st = launch_cfg<64, 64, false>(a, nt, s);
    }
  }
  if (st || p.split == 1) return st;
  const int64_t quads = static_cast<int64_t>(a.m) * (p.n_out / 4);
  hipLaunchKernelGGL(nf4_gemm_reduce, dim3(static_cast<uint32_t>((quads + 255) / 256)), dim3(256),
                     0, s, a.ws, p.split, a.m, p.n_out, bias, out, ldo, a.out32);
  return cm::launch_status();
}

int fwd_args(const void* x, int64_t ldx, int64_t m, const cm_nf4_weight* w, int n_w, Args& a) {
  if (int st = setup(w, n_w, m, a)) return st;
  if (m > 0) CM_CHECK_ARG(x && cm::aligned(x, 16) && ldx >= a.cols && ldx % 8 == 0);
  a.x = static_cast<const _Float16*>(x);
  a.ldx = ldx;
  return 0;
}

int bwd_args(const cm_nf4_weight* w, int n_w, int64_t m, Args& a) {
  if (int st = setup(w, n_w, m, a)) return st;
  int stages = 0;
  for (int i = 0; i < n_w; ++i) {
    a.w[i].first = stages;
    stages += a.w[i].rows / kBK;
  }
  a.n_stages = stages;
  return 0;
}

}  // namespace

extern "C" int cm_nf4_scale_map(const cm_nf4_weight* w, float* smap, void* stream) {
  Args a;
  if (int st = setup(w, 1, 0, a)) return st;
  CM_CHECK_ARG(smap && cm::aligned(smap, 16) && a.cols % w->blocksize == 0);
  const int64_t n = static_cast<int64_t>(a.cols / w->blocksize) * a.w[0].rows;
  CM_CHECK_ARG((n + 255) / 256 < 0x7fffffff);
  hipLaunchKernelGGL(nf4_scale_map_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), a.w[0], a.nested, a.cols,
                     smap);
  return cm::launch_status();
}

extern "C" int64_t cm_nf4_linear_workspace_bytes(int64_t m, const cm_nf4_weight* w, int n_w,
                                                 int backward) {
  Args a;
  if (setup(w, n_w, m, a)) return -1;
  if (m == 0) return 0;
  if (backward) {
    bwd_args(w, n_w, m, a);
    return plan_for(a, true).ws_bytes;
  }
  return plan_for(a, false).ws_bytes;
}

extern "C" int cm_nf4_linear_fwd(const void* x, int64_t ldx, int64_t m, const cm_nf4_weight* w,
                                 int n_w, const void* const* bias, void* const* out,
                                 const int64_t* ldo, int out_dtype, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  Args a;
  CM_CHECK_ARG(out_dtype == CM_F16 || out_dtype == CM_F32);
  CM_CHECK_ARG(out != nullptr && ldo != nullptr);
  if (int st = fwd_args(x, ldx, m, w, n_w, a)) return st;
  if (m == 0) return 0;
  a.out32 = out_dtype == CM_F32;
  for (int i = 0; i < n_w; ++i) {
    WeightDev& d = a.w[i];
    CM_CHECK_ARG(out[i] && ldo[i] >= d.rows && ldo[i] % 4 == 0);
    CM_CHECK_ARG(cm::aligned(out[i], a.out32 ? 16 : 8));
    d.out = out[i];
    d.ldo = ldo[i];
    d.bias = bias ? static_cast<const _Float16*>(bias[i]) : nullptr;
    if (d.bias) CM_CHECK_ARG(cm::aligned(d.bias, 8));
  }
  const Plan p = plan_for(a, false);
  return run(a, p, false, workspace, workspace_bytes, a.w[0].out, a.w[0].ldo, a.w[0].bias,
             static_cast<hipStream_t>(stream));
}

extern "C" int cm_nf4_linear_bwd(const void* const* g, const int64_t* ldg, int64_t m,
                                 const cm_nf4_weight* w, int n_w, void* dx, int64_t lddx,
                                 int dx_dtype, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  Args a;
  CM_CHECK_ARG(dx_dtype == CM_F16 || dx_dtype == CM_F32);
  CM_CHECK_ARG(g != nullptr && ldg != nullptr);
  if (int st = bwd_args(w, n_w, m, a)) return st;
  if (m == 0) return 0;
  a.out32 = dx_dtype == CM_F32;
  CM_CHECK_ARG(dx && lddx >= a.cols && lddx % 4 == 0 && cm::aligned(dx, a.out32 ? 16 : 8));
  a.dx = dx;
  a.lddx = lddx;
  for (int i = 0; i < n_w; ++i) {
    WeightDev& d = a.w[i];
    CM_CHECK_ARG(g[i] && cm::aligned(g[i], 16) && ldg[i] >= d.rows && ldg[i] % 8 == 0);
    d.g = static_cast<const _Float16*>(g[i]);
    d.ldg = ldg[i];
  }
  const Plan p = plan_for(a, true);
  return run(a, p, true, workspace, workspace_bytes, dx, lddx, nullptr,
             static_cast<hipStream_t>(stream));
}
