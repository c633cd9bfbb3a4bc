// NF4 dequantization with the nested absmax decoded in the same pass (gfx950).
//
// Reproduces solution/nf4.py:26-46 (nf4_dequant_kernel) bit for bit. Layout: byte i of the
// packed weight holds element 2i in its high nibble and 2i+1 in its low nibble; element j
// belongs to absmax block j / blocksize. With double quantization the block scale is
// code2[absmax8[b]] * absmax2[b / blocksize2] + offset, an fp32 multiply followed by an fp32
// add (nf4.py:37-38, compiled there with fp fusion off). Each output is the fp32 product
// code[nibble] * scale rounded to nearest even in the output type.
//
// Work split: a lane handles 4-byte units (8 outputs, one 16-byte fp16 store), all 8 in one
// absmax block because blocksize >= 32. A workgroup of 256 lanes handles UNITS consecutive
// 1 KiB slices of the packed weight, so every load and store instruction of a wavefront covers
// one contiguous span (256 B in, 1 KiB out for fp16). The fp16 outputs go out as nontemporal
// stores (measured on MI355X: 8.7 -> 7.5 us on the [8960,1536] weight, cold
// caches). The code table sits in LDS as 256 pairs (code[b >> 4], code[b & 15]), one per packed
// byte value b, so a byte's two code values are one 8-byte lookup indexed by the byte itself.
#include "common.h"

namespace {

// No contraction anywhere in this file's arithmetic: the scale is a multiply then an add.
#pragma clang fp contract(off)

constexpr int kThreads = 256;
constexpr int kUnits = 4;  // 4-byte units per lane
constexpr int64_t kResidentBlocks = 2048;  // 256-lane workgroups the chip holds at once

template <bool NESTED>
__device__ __forceinline__ float block_scale(const void* absmax, const float* code2,
                                             const float* absmax2, float offset, uint32_t blk,
                                             int bs2_shift, uint32_t bs2) {
  if constexpr (NESTED) {
    const uint8_t q8 = static_cast<const uint8_t*>(absmax)[blk];
    const uint32_t blk2 = bs2_shift >= 0 ? (blk >> bs2_shift) : (blk / bs2);
    const float prod = code2[q8] * absmax2[blk2];
    return prod + offset;
  } else {
    return static_cast<const float*>(absmax)[blk];
  }
}

template <typename OutT>
struct Pack8;

template <>
struct Pack8<_Float16> {
  static __device__ __forceinline__ void store(_Float16* out, const float (&v)[8]) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = cm::from_f32<_Float16>(v[i]);
    __builtin_nontemporal_store(h, reinterpret_cast<h8*>(out));
  }
};

template <>
struct Pack8<cm::bf16_t> {
  static __device__ __forceinline__ void store(cm::bf16_t* out, const float (&v)[8]) {
    uint4 r;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = static_cast<uint32_t>(cm::from_f32<cm::bf16_t>(v[2 * i]).bits) |
             (static_cast<uint32_t>(cm::from_f32<cm::bf16_t>(v[2 * i + 1]).bits) << 16);
    }
    r.x = w[0]; r.y = w[1]; r.z = w[2]; r.w = w[3];
    *reinterpret_cast<uint4*>(out) = r;
  }
};

template <>
struct Pack8<float> {
  static __device__ __forceinline__ void store(float* out, const float (&v)[8]) {
    float4 a = make_float4(v[0], v[1], v[2], v[3]);
    float4 b = make_float4(v[4], v[5], v[6], v[7]);
    reinterpret_cast<float4*>(out)[0] = a;
    reinterpret_cast<float4*>(out)[1] = b;
  }
};

// Vector path: packed 4-byte aligned, out 16-byte aligned. Units [0, n_units) of 4 bytes. A
// workgroup's 1024 units span at most 256 absmax blocks (blocksize >= 32 elements = 4 units), and
// lane t stages block blk0 + t in LDS: its absmax byte and absmax2 entry (or its fp32 absmax),
// with one entry of the 256-entry code2 table and one of the 256 code pairs per lane. Those
// loads are issued first, then the lane's packed words; one barrier, after which a unit's scale
// is code2[q8] * absmax2 + offset from LDS and each of its bytes one pair lookup (a lookup per
// nibble and the nibble arithmetic took 201 VALU instructions and 40 LDS reads per lane, the
// pairs 158 and 24: 6.8-7.0 -> 6.6 us at [8960,1536], same process, bit-identical). Workgroups
// whose units all lie inside the weight (all but the last) skip the per-unit bounds tests
// (-0.1 us). A lane thus issues its 4 word loads and at most 3
// coalesced others (loading the absmax byte and absmax2 entry per unit took 12, and the kernel
// 7.2 us at [8960,1536] against 6.0 us for the same loads and stores without the decode; now
// 6.7 us). SCALES_FIRST issues the block loads before the packed words: faster when every
// workgroup of the launch is resident at once (the barrier waits on the earliest loads), slower
// by ~3% for a streaming launch of many waves of workgroups, which issues the words first.
// Both orders compute the same values.
// The workgroup body, for workgroup `wg` of one weight's launch (the single-weight kernel and the
// grouped one both run it).
template <typename OutT, bool NESTED, bool SCALES_FIRST>
__device__ __forceinline__ void dequant_vec_wg(
    const uint32_t* __restrict__ packed, const void* __restrict__ absmax,
    const float* __restrict__ code, const float* __restrict__ code2,
    const float* __restrict__ absmax2, const float* __restrict__ offset_ptr,
    OutT* __restrict__ out, int64_t n_units, int unit_shift, int bs2_shift, uint32_t bs2,
    uint32_t wg) {
  static_assert(kThreads >= 256, "one code2 entry per lane");
  static_assert(kThreads * kUnits / 4 <= kThreads, "one absmax block of the range per lane");
  static_assert(kThreads == 256, "one code pair per lane");
  __shared__ float2 s_pair[256];  // packed byte b -> (code[b >> 4], code[b & 15])
  __shared__ float s_code2[NESTED ? 256 : 1];
  __shared__ uint2 s_blk[kThreads];  // block blk0 + t: {absmax byte, absmax2 bits} or {-, absmax}
  const int t = threadIdx.x;
  const int64_t u0 = static_cast<int64_t>(wg) * (kThreads * kUnits);
  const uint32_t blk0 = static_cast<uint32_t>(u0 >> unit_shift);
  // blocks in the workgroup's range (1 when the range lies inside one block)
  const int nb = unit_shift < 30 && ((kThreads * kUnits) >> unit_shift) > 0
                     ? (kThreads * kUnits) >> unit_shift
                     : 1;
  uint32_t q8 = 0;
  float a2 = 0.0f, c2 = 0.0f;
  uint32_t word[kUnits];
  auto load_words = [&] {
#pragma unroll
    for (int j = 0; j < kUnits; ++j) {
      const int64_t u = u0 + t + j * kThreads;
      word[j] = u < n_units ? __builtin_nontemporal_load(packed + u) : 0u;
    }
  };
  if constexpr (!SCALES_FIRST) load_words();
  if (t < nb) {
    const uint32_t blk = blk0 + t;
    if ((static_cast<int64_t>(blk) << unit_shift) < n_units) {
      if constexpr (NESTED) {
        q8 = static_cast<const uint8_t*>(absmax)[blk];
        a2 = absmax2[bs2_shift >= 0 ? (blk >> bs2_shift) : (blk / bs2)];
      } else {
        a2 = static_cast<const float*>(absmax)[blk];
      }
    }
  }
  const float2 pair = make_float2(code[t >> 4], code[t & 15]);
  if constexpr (NESTED) c2 = code2[t];
  if constexpr (SCALES_FIRST) load_words();
  if (t < nb) s_blk[t] = uint2{q8, __builtin_bit_cast(uint32_t, a2)};
  s_pair[t] = pair;
  if constexpr (NESTED) s_code2[t] = c2;
  const float offset = NESTED ? *offset_ptr : 0.0f;
  __syncthreads();
  auto unit = [&](int j) {
    const int64_t u = u0 + t + j * kThreads;
    const uint2 e = s_blk[static_cast<uint32_t>(u >> unit_shift) - blk0];
    float s;
    if constexpr (NESTED) {
      const float prod = s_code2[e.x] * __builtin_bit_cast(float, e.y);  // multiply, then add
      s = prod + offset;
    } else {
      s = __builtin_bit_cast(float, e.y);
    }
    float v[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float2 cp = s_pair[(word[j] >> (8 * k)) & 0xffu];  // high nibble first
      v[2 * k] = cp.x * s;
      v[2 * k + 1] = cp.y * s;
    }
    Pack8<OutT>::store(out + 8 * u, v);
  };
  if (u0 + kThreads * kUnits <= n_units) {  // every workgroup but the last: no bounds tests
#pragma unroll
    for (int j = 0; j < kUnits; ++j) unit(j);
  } else {
#pragma unroll
    for (int j = 0; j < kUnits; ++j)
      if (u0 + t + j * kThreads < n_units) unit(j);
  }
}

template <typename OutT, bool NESTED, bool SCALES_FIRST>
__global__ __launch_bounds__(kThreads) void nf4_dequant_vec(
    const uint32_t* __restrict__ packed, const void* __restrict__ absmax,
    const float* __restrict__ code, const float* __restrict__ code2,
    const float* __restrict__ absmax2, const float* __restrict__ offset_ptr,
    OutT* __restrict__ out, int64_t n_units, int unit_shift, int bs2_shift, uint32_t bs2) {
  dequant_vec_wg<OutT, NESTED, SCALES_FIRST>(packed, absmax, code, code2, absmax2, offset_ptr,
                                             out, n_units, unit_shift, bs2_shift, bs2,
                                             blockIdx.x);
}

// Several weights expanded by one launch: weight i takes workgroups [first[i], first[i + 1]) and
// each workgroup runs the single-weight body on its weight, so every output element is the one
// the single-weight kernel writes. A workgroup finds its weight with static indices only (the
// descriptors stay in kernel-argument registers).
constexpr int kGroupMax = 8;
struct DqJob {
  const uint32_t* packed;
  const void* absmax;
  const float* code;
  const float* code2;
  const float* absmax2;
  const float* offset;
  void* out;
  int64_t n_units;
  int unit_shift, bs2_shift;
  uint32_t bs2;
};
struct DqGroup {
  DqJob job[kGroupMax];
  uint32_t first[kGroupMax];
  int n;
};

template <typename OutT, bool NESTED>
__global__ __launch_bounds__(kThreads) void nf4_dequant_group(DqGroup g) {
  const uint32_t b = blockIdx.x;
  DqJob job = g.job[0];
  uint32_t first = 0;
#pragma unroll
  for (int i = 1; i < kGroupMax; ++i) {
    if (i < g.n && b >= g.first[i]) {
      job = g.job[i];
      first = g.first[i];
    }
  }
  dequant_vec_wg<OutT, NESTED, false>(job.packed, job.absmax, job.code, job.code2, job.absmax2,
                                      job.offset, static_cast<OutT*>(job.out), job.n_units,
                                      job.unit_shift, job.bs2_shift, job.bs2, b - first);
}

// Scalar path: one packed byte per lane, any alignment; bytes [first, n_bytes).
template <typename OutT, bool NESTED>
__global__ __launch_bounds__(kThreads) void nf4_dequant_bytes(
    const uint8_t* __restrict__ packed, const void* __restrict__ absmax,
    const float* __restrict__ code, const float* __restrict__ code2,
    const float* __restrict__ absmax2, const float* __restrict__ offset_ptr,
    OutT* __restrict__ out, int64_t first, int64_t n_bytes, int byte_shift, int bs2_shift,
    uint32_t bs2) {
  const int64_t i = first + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n_bytes) return;
  const float offset = NESTED ? *offset_ptr : 0.0f;
  const uint32_t byte = packed[i];
  const uint32_t blk = static_cast<uint32_t>(i >> byte_shift);  // blocksize/2 bytes per block
  const float s = block_scale<NESTED>(absmax, code2, absmax2, offset, blk, bs2_shift, bs2);
  out[2 * i] = cm::from_f32<OutT>(code[byte >> 4] * s);
  out[2 * i + 1] = cm::from_f32<OutT>(code[byte & 0xfu] * s);
}

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

template <typename OutT, bool NESTED>
int launch(const uint8_t* packed, const void* absmax, const float* code, const float* code2,
           const float* absmax2, const float* offset, void* out_v, int64_t n_bytes,
           int blocksize, int blocksize2, hipStream_t stream) {
  OutT* out = static_cast<OutT*>(out_v);
  const int bs_shift = log2_exact(blocksize);
  const int bs2_shift = log2_exact(blocksize2);
  int64_t done = 0;
  const bool vec = cm::aligned(packed, 4) && cm::aligned(out, 16);
  if (vec) {
    const int64_t n_units = n_bytes / 4;
    if (n_units > 0) {
      const int64_t per_block = int64_t{kThreads} * kUnits;
      const int64_t blocks = (n_units + per_block - 1) / per_block;
      if (blocks > 0x7fffffff) return static_cast<int>(hipErrorInvalidValue);
      // unit u covers elements [8u, 8u+8): block index = 8u / blocksize = u >> (bs_shift - 3)
      // one wave of resident workgroups (256 CUs x 8) or fewer: latency-bound, block loads first
      auto kern = blocks <= kResidentBlocks ? nf4_dequant_vec<OutT, NESTED, true>
                                            : nf4_dequant_vec<OutT, NESTED, false>;
      hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream,
                         reinterpret_cast<const uint32_t*>(packed), absmax, code, code2,
                         absmax2, offset, out, n_units, bs_shift - 3, bs2_shift,
                         static_cast<uint32_t>(blocksize2));
      int st = cm::launch_status();
      if (st) return st;
    }
    done = n_units * 4;
  }
  const int64_t rest = n_bytes - done;
  if (rest > 0) {
    const int64_t blocks = (rest + kThreads - 1) / kThreads;
    if (blocks > 0x7fffffff) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL((nf4_dequant_bytes<OutT, NESTED>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(kThreads), 0, stream, packed, absmax, code, code2, absmax2, offset,
                       out, done, n_bytes, bs_shift - 1, bs2_shift,
                       static_cast<uint32_t>(blocksize2));
    int st = cm::launch_status();
    if (st) return st;
  }
  return 0;
}

}  // namespace

namespace {

// Transposed expansion, fp16 only: out[c][r] = W[r][c] for W [rows, cols], rows a multiple of
// 64 and cols of 128. A workgroup of 256 lanes expands a 64 x 128 tile through the LDS:
//  - lane task p = t + 256 j (j < 2) decodes packed word wc = p % 16 (columns 8 wc .. +7 of the
//    tile, one absmax block since blocksize >= 32) of the rows 2 rp and 2 rp + 1, rp = p / 16,
//    so a load instruction covers 4 rows x 64 contiguous bytes;
//  - each of the 8 columns gets the two rows as one 32-bit LDS write; columns are 66 halves
//    apart, which spreads a wavefront's writes over 32 banks (16 B-aligned columns of 72
//    halves put them on 4);
//  - after the barrier, lane task q = t + 256 i writes rows 8 part .. +7 and 32 + 8 part .. +7 of
//    column q / 4 (part = q % 4), so each store instruction writes 64 contiguous bytes of 16
//    columns.
// The values are those of nf4_dequant_vec, bit for bit.
template <bool NESTED>
__global__ __launch_bounds__(kThreads) void nf4_dequant_t_kernel(
    const uint32_t* __restrict__ packed, const void* __restrict__ absmax,
    const float* __restrict__ code, const float* __restrict__ code2,
    const float* __restrict__ absmax2, const float* __restrict__ offset_ptr,
    _Float16* __restrict__ out, int64_t rows, int64_t cols, int unit_shift, int bs2_shift,
    uint32_t bs2) {
  constexpr int kTR = 64, kTC = 128, kCol = (kTR + 2) / 2;  // 32-bit words per LDS column
  __shared__ float s_code[16];
  __shared__ float s_scale[kTR * (kTC / 32)];  // [row][block of the row's 128 columns]
  __shared__ uint32_t tile[kTC * kCol];  // [column][row pair]
  const int64_t tiles_c = cols / kTC;
  const int64_t r0 = (blockIdx.x / tiles_c) * kTR, c0 = (blockIdx.x % tiles_c) * kTC;
  uint32_t word[2][2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = threadIdx.x + kThreads * j, rp = p / 16, wc = p % 16;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t unit = ((r0 + 2 * rp + h) * cols + c0) / 8 + wc;  // 8 elements per unit
      word[j][h] = __builtin_nontemporal_load(packed + unit);
    }
  }
  if (threadIdx.x < 16) s_code[threadIdx.x] = code[threadIdx.x];
  const float offset = NESTED ? *offset_ptr : 0.0f;
  // The tile's block scales, decoded once: a row's 128 columns start at a multiple of 128 and
  // hold nb = max(1, 128 / blocksize) whole blocks (or lie inside one).
  const int nb = max(1, (kTC / 8) >> unit_shift);
  if (threadIdx.x < kTR * nb) {
    const int r = threadIdx.x / nb, k = threadIdx.x % nb;
    const uint32_t blk = static_cast<uint32_t>((((r0 + r) * cols + c0) / 8 >> unit_shift) + k);
    s_scale[threadIdx.x] = block_scale<NESTED>(absmax, code2, absmax2, offset, blk, bs2_shift, bs2);
  }
  __syncthreads();  // s_code, s_scale
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = threadIdx.x + kThreads * j, rp = p / 16, wc = p % 16;
    uint32_t lo[8], hi[8];  // fp16 bits of the 8 columns, rows 2 rp and 2 rp + 1
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float sc = s_scale[(2 * rp + h) * nb + (wc >> unit_shift)];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t byte = (word[j][h] >> (8 * k)) & 0xffu;
        const uint32_t a = __builtin_bit_cast(uint16_t, cm::from_f32<_Float16>(s_code[byte >> 4] * sc));
        const uint32_t b = __builtin_bit_cast(uint16_t, cm::from_f32<_Float16>(s_code[byte & 0xfu] * sc));
        (h ? hi : lo)[2 * k] = a;
        (h ? hi : lo)[2 * k + 1] = b;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[(8 * wc + e) * kCol + rp] = lo[e] | (hi[e] << 16);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = threadIdx.x + kThreads * i, col = q / 4, part = q % 4;
    const uint32_t* src = tile + col * kCol;
    _Float16* dst = out + (c0 + col) * rows + r0;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int w0 = 16 * half + 4 * part;  // row pair of row 32 half + 8 part
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 v = {src[w0], src[w0 + 1], src[w0 + 2], src[w0 + 3]};
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + 32 * half + 8 * part));
    }
  }
}

}  // namespace

// Transposed expansion for the MLP backward (no counterpart in the reference: its input
// gradient multiplies by the expanded weight as stored).
extern "C" int cm_nf4_dequant_t(const uint8_t* packed, const void* absmax, int nested,
                                const float* code, const float* code2, const float* absmax2,
                                const float* offset, void* out, int64_t rows, int64_t cols,
                                int blocksize, int blocksize2, void* stream) {
  CM_CHECK_ARG(rows >= 0 && cols >= 0 && rows % 64 == 0 && cols % 128 == 0);
  if (rows == 0 || cols == 0) return 0;
  CM_CHECK_ARG(packed && absmax && code && out);
  CM_CHECK_ARG((reinterpret_cast<uintptr_t>(packed) & 3) == 0 &&
               (reinterpret_cast<uintptr_t>(out) & 15) == 0);
  CM_CHECK_ARG(blocksize >= 32 && log2_exact(blocksize) >= 0);
  CM_CHECK_ARG(rows * cols / blocksize < (int64_t{1} << 31));
  CM_CHECK_ARG(rows / 64 * (cols / 128) < (int64_t{1} << 31));
  if (nested) CM_CHECK_ARG(code2 && absmax2 && offset && blocksize2 >= 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int unit_shift = log2_exact(blocksize) - 3;
  const int bs2_shift = nested ? log2_exact(blocksize2) : 0;
  const dim3 grid(static_cast<unsigned>(rows / 64 * (cols / 128)));
  const auto* words = reinterpret_cast<const uint32_t*>(packed);
  if (nested) {
    hipLaunchKernelGGL(nf4_dequant_t_kernel<true>, grid, dim3(kThreads), 0, s, words, absmax,
                       code, code2, absmax2, offset, static_cast<_Float16*>(out), rows, cols,
                       unit_shift, bs2_shift, static_cast<uint32_t>(blocksize2));
  } else {
    hipLaunchKernelGGL(nf4_dequant_t_kernel<false>, grid, dim3(kThreads), 0, s, words, absmax,
                       code, nullptr, nullptr, nullptr, static_cast<_Float16*>(out), rows, cols,
                       unit_shift, 0, 1u);
  }
  return cm::launch_status();
}

extern "C" int cm_nf4_dequant(const uint8_t* packed, const void* absmax, int nested,
                              const float* code, const float* code2, const float* absmax2,
                              const float* offset, void* out, int out_dtype, int64_t n_bytes,
                              int blocksize, int blocksize2, void* stream) {
  CM_CHECK_ARG(n_bytes >= 0);
  if (n_bytes == 0) return 0;
  CM_CHECK_ARG(packed && absmax && code && out);
  CM_CHECK_ARG(blocksize >= 32 && log2_exact(blocksize) >= 0);
  // absmax block indices are 32-bit: n_bytes * 2 / blocksize must fit
  CM_CHECK_ARG(n_bytes / (blocksize / 2) < (int64_t{1} << 31));
  if (nested) CM_CHECK_ARG(code2 && absmax2 && offset && blocksize2 >= 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define CM_NF4_CASE(T)                                                                        \
  return nested ? launch<T, true>(packed, absmax, code, code2, absmax2, offset, out, n_bytes, \
                                  blocksize, blocksize2, s)                                   \
                : launch<T, false>(packed, absmax, code, code2, absmax2, offset, out,         \
                                   n_bytes, blocksize, 1, s)
  switch (out_dtype) {
    case CM_F16: CM_NF4_CASE(_Float16);
    case CM_F32: CM_NF4_CASE(float);
    case CM_BF16: CM_NF4_CASE(cm::bf16_t);
    default: return static_cast<int>(hipErrorInvalidValue);
  }
#undef CM_NF4_CASE
}

namespace {

// Whether cm_nf4_dequant_group can take the weights in one launch: the vector path for every
// weight (4-byte aligned packed bytes in whole 4-byte units, 16-byte aligned outputs), one
// nestedness, power-of-two block sizes.
bool groupable(const cm_nf4_weight* w, int n_w, void* const* out) {
  for (int i = 0; i < n_w; ++i) {
    const int64_t n_bytes = w[i].rows * w[i].cols / 2;
    if (w[i].nested != w[0].nested || n_bytes % 4 || !cm::aligned(w[i].packed, 4) ||
        !cm::aligned(out[i], 16))
      return false;
  }
  return true;
}

template <typename OutT, bool NESTED>
int launch_group(const cm_nf4_weight* w, int n_w, void* const* out, hipStream_t s) {
  DqGroup g{};
  int64_t blocks = 0;
  const int64_t per_block = int64_t{kThreads} * kUnits;
  for (int i = 0; i < n_w; ++i) {
    const int64_t n_units = w[i].rows * w[i].cols / 8;
    g.first[i] = static_cast<uint32_t>(blocks);
    g.job[i] = DqJob{reinterpret_cast<const uint32_t*>(w[i].packed), w[i].absmax, w[i].code,
                     NESTED ? w[i].code2 : nullptr, NESTED ? w[i].absmax2 : nullptr,
                     NESTED ? w[i].offset : nullptr, out[i], n_units,
                     log2_exact(w[i].blocksize) - 3,
                     NESTED ? log2_exact(w[i].blocksize2) : 0,
                     NESTED ? static_cast<uint32_t>(w[i].blocksize2) : 1u};
    blocks += (n_units + per_block - 1) / per_block;
  }
  g.n = n_w;
  if (blocks == 0) return 0;
  hipLaunchKernelGGL((nf4_dequant_group<OutT, NESTED>), dim3(static_cast<uint32_t>(blocks)),
                     dim3(kThreads), 0, s, g);
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_nf4_dequant_group(const cm_nf4_weight* w, int n_w, void* const* out,
                                    int out_dtype, void* stream) {
  CM_CHECK_ARG(n_w >= 0 && n_w <= kGroupMax);
  if (n_w == 0) return 0;
  CM_CHECK_ARG(w && out);
  int64_t blocks = 0;
  for (int i = 0; i < n_w; ++i) {
    const cm_nf4_weight& d = w[i];
    CM_CHECK_ARG(d.rows >= 0 && d.cols >= 0 && (d.rows * d.cols) % 2 == 0);
    if (d.rows * d.cols == 0) continue;
    CM_CHECK_ARG(d.packed && d.absmax && d.code && out[i]);
    CM_CHECK_ARG(d.blocksize >= 32 && log2_exact(d.blocksize) >= 0);
    CM_CHECK_ARG(d.rows * d.cols / d.blocksize < (int64_t{1} << 31));
    if (d.nested) CM_CHECK_ARG(d.code2 && d.absmax2 && d.offset && d.blocksize2 >= 1);
    blocks += (d.rows * d.cols / 8 + kThreads * kUnits - 1) / (kThreads * kUnits);
  }
  CM_CHECK_ARG(blocks < (int64_t{1} << 31));
  CM_CHECK_ARG(out_dtype == CM_F16 || out_dtype == CM_F32 || out_dtype == CM_BF16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // empty weights are left out of the launch
  cm_nf4_weight ws[kGroupMax];
  void* outs[kGroupMax];
  int n = 0;
  for (int i = 0; i < n_w; ++i) {
    if (w[i].rows * w[i].cols == 0) continue;
    ws[n] = w[i];
    outs[n++] = out[i];
  }
  if (n == 0) return 0;
  if (!groupable(ws, n, outs)) {  // one launch per weight, the same kernels and values
    for (int i = 0; i < n; ++i) {
      const cm_nf4_weight& d = ws[i];
      const int st = cm_nf4_dequant(d.packed, d.absmax, d.nested, d.code, d.code2, d.absmax2,
                                    d.offset, outs[i], out_dtype, d.rows * d.cols / 2,
                                    d.blocksize, d.nested ? d.blocksize2 : 1, stream);
      if (st) return st;
    }
    return 0;
  }
#define CM_NF4_GROUP(T)                                                  \
  return ws[0].nested ? launch_group<T, true>(ws, n, outs, s)            \
                      : launch_group<T, false>(ws, n, outs, s)
  switch (out_dtype) {
    case CM_F16: CM_NF4_GROUP(_Float16);
    case CM_F32: CM_NF4_GROUP(float);
    default: CM_NF4_GROUP(cm::bf16_t);
  }
#undef CM_NF4_GROUP
}
