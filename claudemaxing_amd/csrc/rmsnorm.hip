// RMSNorm of Qwen2, forward and backward (gfx950).
//
// Reproduces solution/rmsnorm.py:28-47 (qwen_rmsnorm_fwd_kernel) and 51-91
// (qwen_rmsnorm_bwd_kernel):
//   rstd = 1 / sqrt(sum(x^2) / n + eps)      fp32
//   normed = round_x(x * rstd);  out = round_out(normed * w)
//   backward: gn = round_x(dy * w) (not rounded on the saved-output path),
//             dx = round_x((gn - normed * sum(gn * normed) / n) * rstd),
//             dw partial += dy * round_x(normed)
// with the SAVE_LOW variant (fp32 x, frozen fp32 w) that keeps only the fp16 copy of the output
// and the fp16 normalised values of the tiny-|w| columns, from which backward rebuilds normed.
//
// The residual variants fuse the adds of Qwen2's decoder layer (transformers'
// Qwen2DecoderLayer.forward: h = residual + attention output, then the norm of h) into the norm:
// the forward computes and writes h = residual + x (fp32) before normalising it, and the backward
// adds the residual's gradient to the norm's input gradient (dh = dres + dx, the sum autograd
// forms where the two uses of h meet) and may write the fp16 copy of dh that the projection
// before it casts its gradient to. Both adds are separate fp32 roundings, as torch's adds are.
//
// One wavefront owns one row; the row's sums are 64-lane shuffle reductions (no LDS, no block
// barrier). A lane holds NV vectors of VEC contiguous columns in registers (VEC = 8: one
// 16-byte access per vector for fp16), so x is read from HBM once; for rows wider than
// NV * 64 * VEC columns the lane loops and the second pass re-reads the row from cache
// (NV = 0). Four rows per 256-lane workgroup.
#include <type_traits>

#include "vec.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / cm::kWave;
constexpr int kMaxBwdBlocks = 512;

// a + b rounded on its own: never contracted with a product that feeds it (torch's fp32 add)
__device__ __forceinline__ float add_alone(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

template <typename T, int VEC>
__device__ __forceinline__ void load_v(const T* p, float (&v)[VEC], int cnt) {
  if constexpr (VEC == 8) {
    cm::Vec8<T, true>::load(p, v, cnt);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = i < cnt ? cm::to_f32(p[i]) : 0.0f;
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_v(T* p, const float (&v)[VEC], int cnt) {
  if constexpr (VEC == 8) {
    cm::Vec8<T, true>::store(p, v, cnt);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      if (i < cnt) p[i] = cm::from_f32<T>(v[i]);
  }
}

// NV > 0: the lane's columns are cached in registers; NV == 0: loop over the row.
template <typename XT, typename WT, typename OT, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_kernel(
    const XT* __restrict__ x, int64_t x_stride, const WT* __restrict__ w, OT* __restrict__ out,
    float* __restrict__ rstd, _Float16* __restrict__ low16, const int32_t* __restrict__ slot,
    _Float16* __restrict__ small16, int n_small, int64_t n_rows, int n_cols, float eps) {
  const int lane = threadIdx.x % cm::kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / cm::kWave;
  if (row >= n_rows) return;
  const XT* xr = x + row * x_stride;
  OT* orow = out + row * static_cast<int64_t>(n_cols);
  constexpr int kCache = NV > 0 ? NV : 1;
  float xv[kCache][VEC];
  float ss = 0.0f;
  const int step = cm::kWave * VEC;
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = i * step + lane * VEC;
      const int cnt = c < n_cols ? min(VEC, n_cols - c) : 0;
      load_v<XT, VEC>(xr + c, xv[i], cnt);
#pragma unroll
      for (int k = 0; k < VEC; ++k) ss += xv[i][k] * xv[i][k];
    }
  } else {
    for (int c = lane * VEC; c < n_cols; c += step) {
      load_v<XT, VEC>(xr + c, xv[0], min(VEC, n_cols - c));
#pragma unroll
      for (int k = 0; k < VEC; ++k) ss += xv[0][k] * xv[0][k];
    }
  }
  ss = cm::wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(n_cols) + eps);
  if (lane == 0) rstd[row] = r;
  const bool save_low = low16 != nullptr;
  const bool any_small = save_low && n_small > 0;  // else the column map is not read at all
  const int n_iter = NV > 0 ? NV : (n_cols + step - 1) / step;
  for (int i = 0; i < n_iter; ++i) {
    const int c = i * step + lane * VEC;
    if (c >= n_cols) break;
    const int cnt = min(VEC, n_cols - c);
    float xi[VEC], wv[VEC], o[VEC], nv[VEC];
    if constexpr (NV > 0) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) xi[k] = xv[i][k];
    } else {
      load_v<XT, VEC>(xr + c, xi, cnt);
    }
    load_v<WT, VEC>(w + c, wv, cnt);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      nv[k] = cm::round_to<XT>(xi[k] * r);  // rounded to the input dtype before the weight
      o[k] = nv[k] * wv[k];
    }
    store_v<OT, VEC>(orow + c, o, cnt);
    if (save_low) {
      store_v<_Float16, VEC>(low16 + row * static_cast<int64_t>(n_cols) + c, o, cnt);
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        if (any_small && k < cnt) {
          const int sl = slot[c + k];
          if (sl >= 0) small16[row * static_cast<int64_t>(n_small) + sl] =
              cm::from_f32<_Float16>(nv[k]);
        }
      }
    }
  }
}

// Persistent over rows: wave g handles rows g, g + n_waves, ... and (with dw_partial) writes its
// partial dw row g, zeros if it had no row.
template <typename DT, typename XT, typename WT, typename DXT, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_kernel(
    const DT* __restrict__ dy, const void* __restrict__ xs_v, const WT* __restrict__ w,
    const float* __restrict__ rstd, DXT* __restrict__ dx, float* __restrict__ dw_partial,
    const int32_t* __restrict__ slot, const _Float16* __restrict__ small16, int n_small,
    int saved_output, int64_t n_rows, int n_cols) {
  const int lane = threadIdx.x % cm::kWave;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / cm::kWave;
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  const int step = cm::kWave * VEC;
  constexpr int kCache = NV > 0 ? NV : 1;
  const bool want_dw = dw_partial != nullptr;
  // Saved-output rows hold fp16 copies of the output; otherwise the rows hold x (type XT).
  const XT* xs = static_cast<const XT*>(xs_v);
  const _Float16* lows = static_cast<const _Float16*>(xs_v);
  float dwacc[kCache][VEC];
#pragma unroll
  for (int i = 0; i < kCache; ++i)
#pragma unroll
    for (int k = 0; k < VEC; ++k) dwacc[i][k] = 0.0f;

  for (int64_t row = wave; row < n_rows; row += n_waves) {
    const float r = rstd[row];
    const DT* dyr = dy + row * static_cast<int64_t>(n_cols);
    float nc[kCache][VEC], gc[kCache][VEC];
    float dot = 0.0f;
    const int n_iter = NV > 0 ? NV : (n_cols + step - 1) / step;
    // pass 1: normed and grad_normed, their dot product
    for (int i = 0; i < n_iter; ++i) {
      const int c = i * step + lane * VEC;
      const int cnt = c < n_cols ? min(VEC, n_cols - c) : 0;
      if (NV == 0 && cnt == 0) break;
      const int ci = NV > 0 ? i : 0;
      float d[VEC], wv[VEC], xv[VEC], nv[VEC], gv[VEC];
      load_v<DT, VEC>(dyr + c, d, cnt);
      load_v<WT, VEC>(w + c, wv, cnt);
      if (saved_output) {
        load_v<_Float16, VEC>(lows + row * static_cast<int64_t>(n_cols) + c, xv, cnt);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const int sl = (n_small > 0 && k < cnt) ? slot[c + k] : -1;  // no map: not read
          nv[k] = sl >= 0 ? static_cast<float>(small16[row * static_cast<int64_t>(n_small) + sl])
                          : (k < cnt ? xv[k] / wv[k] : 0.0f);
          gv[k] = d[k] * wv[k];
        }
      } else {
        load_v<XT, VEC>(xs + row * static_cast<int64_t>(n_cols) + c, xv, cnt);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          nv[k] = xv[k] * r;
          gv[k] = cm::round_to<XT>(d[k] * wv[k]);
          if (want_dw) dwacc[ci][k] += d[k] * cm::round_to<XT>(nv[k]);
        }
      }
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        dot += gv[k] * nv[k];
        nc[ci][k] = nv[k];
        gc[ci][k] = gv[k];
      }
      if constexpr (NV == 0) {
        // no register cache: finish nothing here, pass 2 recomputes
      }
    }
    dot = cm::wave_sum(dot);
    const float mean_dot = dot / static_cast<float>(n_cols);
    DXT* dxr = dx + row * static_cast<int64_t>(n_cols);
    // pass 2: dx
    for (int i = 0; i < n_iter; ++i) {
      const int c = i * step + lane * VEC;
      if (c >= n_cols) break;
      const int cnt = min(VEC, n_cols - c);
      float nv[VEC], gv[VEC], o[VEC];
      if constexpr (NV > 0) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          nv[k] = nc[i][k];
          gv[k] = gc[i][k];
        }
      } else {
        float d[VEC], wv[VEC], xv[VEC];
        load_v<DT, VEC>(dyr + c, d, cnt);
        load_v<WT, VEC>(w + c, wv, cnt);
        if (saved_output) {
          load_v<_Float16, VEC>(lows + row * static_cast<int64_t>(n_cols) + c, xv, cnt);
#pragma unroll
          for (int k = 0; k < VEC; ++k) {
            const int sl = (n_small > 0 && k < cnt) ? slot[c + k] : -1;
            nv[k] = sl >= 0
                        ? static_cast<float>(small16[row * static_cast<int64_t>(n_small) + sl])
                        : (k < cnt ? xv[k] / wv[k] : 0.0f);
            gv[k] = d[k] * wv[k];
          }
        } else {
          load_v<XT, VEC>(xs + row * static_cast<int64_t>(n_cols) + c, xv, cnt);
#pragma unroll
          for (int k = 0; k < VEC; ++k) {
            nv[k] = xv[k] * r;
            gv[k] = cm::round_to<XT>(d[k] * wv[k]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < VEC; ++k) o[k] = (gv[k] - nv[k] * mean_dot) * r;
      store_v<DXT, VEC>(dxr + c, o, cnt);
    }
  }
  if (want_dw) {
    float* pr = dw_partial + wave * static_cast<int64_t>(n_cols);
    if constexpr (NV > 0) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = i * step + lane * VEC;
        if (c < n_cols) store_v<float, VEC>(pr + c, dwacc[i], min(VEC, n_cols - c));
      }
    } else {
      // Looped rows keep no register cache: redo the sums column by column (rare, wide rows).
      for (int c = lane * VEC; c < n_cols; c += step) {
        const int cnt = min(VEC, n_cols - c);
        float acc[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
        for (int64_t row = wave; row < n_rows; row += n_waves) {
          const float r = rstd[row];
          float d[VEC], xv[VEC];
          load_v<DT, VEC>(dy + row * static_cast<int64_t>(n_cols) + c, d, cnt);
          load_v<XT, VEC>(xs + row * static_cast<int64_t>(n_cols) + c, xv, cnt);
#pragma unroll
          for (int k = 0; k < VEC; ++k) acc[k] += d[k] * cm::round_to<XT>(xv[k] * r);
        }
        store_v<float, VEC>(pr + c, acc, cnt);
      }
    }
  }
}

// Forward for rows of NV * 512 columns: the lane's x vectors and weight vectors are loaded
// together before any arithmetic (one memory round trip per row); with `low16` the fp16 copy of
// the output is written beside it (the case without tiny-|w| columns to keep apart). ADD: the
// norm's input is h = res + x (fp32, written to h), loaded in the same round trip.
template <typename XT, typename WT, typename OT, int NV, bool ADD>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_full_kernel(
    const XT* __restrict__ x, int64_t x_stride, const WT* __restrict__ w, OT* __restrict__ out,
    float* __restrict__ rstd, _Float16* __restrict__ low16, const float* __restrict__ res,
    float* __restrict__ h, int64_t n_rows, int n_cols, float eps) {
  constexpr int VEC = 8;
  using NT = typename std::conditional<ADD, float, XT>::type;  // dtype of the norm's input
  const int lane = threadIdx.x % cm::kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / cm::kWave;
  if (row >= n_rows) return;
  const XT* xr = x + row * x_stride + lane * VEC;
  const int64_t obase = row * static_cast<int64_t>(n_cols) + lane * VEC;
  float xv[NV][VEC], wv[NV][VEC], rv[ADD ? NV : 1][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    cm::Vec8<XT, true>::load(xr + i * cm::kWave * VEC, xv[i]);
    if constexpr (ADD) cm::Vec8<float, true>::load(res + obase + i * cm::kWave * VEC, rv[i]);
    cm::Vec8<WT, true>::load(w + i * cm::kWave * VEC + lane * VEC, wv[i]);
  }
  if constexpr (ADD) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) xv[i][k] = add_alone(rv[i][k], xv[i][k]);
      cm::Vec8<float, true>::store(h + obase + i * cm::kWave * VEC, xv[i]);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int k = 0; k < VEC; ++k) ss += xv[i][k] * xv[i][k];
  ss = cm::wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(n_cols) + eps);
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = cm::round_to<NT>(xv[i][k] * r) * wv[i][k];
    cm::Vec8<OT, true>::store(out + obase + i * cm::kWave * VEC, o);
    if (low16 != nullptr) cm::Vec8<_Float16, true>::store(low16 + obase + i * cm::kWave * VEC, o);
  }
}

// Backward for rows of NV * 512 columns (full 16-byte vectors everywhere), the Qwen2 shapes:
// a wavefront keeps its lane's weight columns in registers across its rows, and issues every
// load of a row (dy, x or the saved fp16 output, rstd) before any arithmetic, so a row costs one
// memory round trip (the general kernel's per-vector length tests made each load wait for the
// previous one). SAVED: xs holds the fp16 copy of the output and normed = copy / w, gn = dy * w
// (the path of fp32 x with a frozen fp32 weight and no tiny-|w| column); otherwise xs holds x,
// normed = x * rstd and gn = round_x(dy * w). POST: dx = dres + (the norm's dx) when dres is
// given (fp32 x), and its fp16 copy to dx16 when that is given.
template <typename DT, typename XT, typename WT, typename DXT, int NV, bool SAVED, bool POST>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_full_kernel(
    const DT* __restrict__ dy, const void* __restrict__ xs_v, const WT* __restrict__ w,
    const float* __restrict__ rstd, DXT* __restrict__ dx, float* __restrict__ dw_partial,
    const float* __restrict__ dres, _Float16* __restrict__ dx16, int64_t n_rows, int n_cols) {
  constexpr int VEC = 8;
  using SrcT = typename std::conditional<SAVED, _Float16, XT>::type;
  const int lane = threadIdx.x % cm::kWave;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / cm::kWave;
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  const SrcT* xs = static_cast<const SrcT*>(xs_v);
  const bool want_dw = dw_partial != nullptr;
  float wv[NV][VEC], dwacc[NV][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    cm::Vec8<WT, true>::load(w + i * cm::kWave * VEC + lane * VEC, wv[i]);
#pragma unroll
    for (int k = 0; k < VEC; ++k) dwacc[i][k] = 0.0f;
  }
  for (int64_t row = wave; row < n_rows; row += n_waves) {
    const int64_t base = row * static_cast<int64_t>(n_cols) + lane * VEC;
    const float r = rstd[row];
    float d[NV][VEC], v[NV][VEC], rg[POST ? NV : 1][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      cm::Vec8<DT, true>::load(dy + base + i * cm::kWave * VEC, d[i]);
      cm::Vec8<SrcT, true>::load(xs + base + i * cm::kWave * VEC, v[i]);
      if constexpr (POST) {
        if (dres != nullptr) cm::Vec8<float, true>::load(dres + base + i * cm::kWave * VEC, rg[i]);
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float nv = SAVED ? v[i][k] / wv[i][k] : v[i][k] * r;
        const float gv = SAVED ? d[i][k] * wv[i][k] : cm::round_to<XT>(d[i][k] * wv[i][k]);
        if (!SAVED && want_dw) dwacc[i][k] += d[i][k] * cm::round_to<XT>(nv);
        dot += gv * nv;
        v[i][k] = nv;
        d[i][k] = gv;
      }
    }
    const float mean_dot = cm::wave_sum(dot) / static_cast<float>(n_cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float o[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) o[k] = (d[i][k] - v[i][k] * mean_dot) * r;
      if constexpr (POST) {
        if (dres != nullptr) {
#pragma unroll
          for (int k = 0; k < VEC; ++k) o[k] = add_alone(rg[i][k], o[k]);
        }
        if (dx16 != nullptr) cm::Vec8<_Float16, true>::store(dx16 + base + i * cm::kWave * VEC, o);
      }
      cm::Vec8<DXT, true>::store(dx + base + i * cm::kWave * VEC, o);
    }
  }
  if (want_dw) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      cm::Vec8<float, true>::store(dw_partial + wave * static_cast<int64_t>(n_cols) +
                                       i * cm::kWave * VEC + lane * VEC,
                                   dwacc[i]);
  }
}

// The residual variants' halves for shapes the full-row kernels do not take: the add before the
// general forward (h = res + x), and the residual gradient after the general backward.
template <typename XT>
__global__ __launch_bounds__(kThreads) void residual_add_kernel(const float* __restrict__ res,
                                                                const XT* __restrict__ x,
                                                                int64_t x_stride,
                                                                float* __restrict__ h,
                                                                int64_t n_rows, int n_cols) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n_rows * n_cols) return;
  const int64_t row = i / n_cols;
  const int64_t col = i - row * n_cols;
  h[i] = add_alone(res[i], cm::to_f32(x[row * x_stride + col]));
}

__global__ __launch_bounds__(kThreads) void residual_grad_kernel(float* __restrict__ dx,
                                                                 const float* __restrict__ dres,
                                                                 _Float16* __restrict__ dx16,
                                                                 int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  float v = dx[i];
  if (dres != nullptr) v = add_alone(dres[i], v);
  dx[i] = v;
  if (dx16 != nullptr) dx16[i] = cm::from_f32<_Float16>(v);
}

// torch.promote_types over the three float dtypes: equal types stay, anything else is fp32
// (fp16 with bf16 promotes to fp32 as well).
int promote(int a, int b) { return a == b ? a : CM_F32; }

template <typename XT, typename WT>
using Promoted = typename std::conditional<std::is_same<XT, WT>::value, XT, float>::type;

int pick_nv(int n_cols, int vec) {
  const int per = cm::kWave * vec;
  const int nv = (n_cols + per - 1) / per;
  (void)vec;
  return nv <= 4 ? nv : 0;
}

int64_t bwd_blocks(int64_t n_rows, bool want_dw) {
  const int64_t need = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
  return want_dw ? (need < kMaxBwdBlocks ? need : kMaxBwdBlocks) : need;
}

#define CM_NV_SWITCH(nv, NV, ...)        \
  switch (nv) {                          \
    case 1: { constexpr int NV = 1; __VA_ARGS__; } break; \
    case 2: { constexpr int NV = 2; __VA_ARGS__; } break; \
    case 3: { constexpr int NV = 3; __VA_ARGS__; } break; \
    case 4: { constexpr int NV = 4; __VA_ARGS__; } break; \
    default: { constexpr int NV = 0; __VA_ARGS__; } break; \
  }

}  // namespace

extern "C" int64_t cm_rmsnorm_bwd_partials(int64_t n_rows) {
  return n_rows <= 0 ? 0 : bwd_blocks(n_rows, true) * kRowsPerBlock;
}

namespace {

// cm_rmsnorm_fwd, and with `res` cm_rmsnorm_add_fwd (the norm of h = res + x, h written).
int fwd_impl(const void* x, int x_dtype, int64_t x_row_stride, const void* w, int w_dtype,
             void* out, int out_dtype, float* rstd, void* low16, const int32_t* slot,
             void* small16, int n_small, int64_t n_rows, int n_cols, float eps, const float* res,
             float* h, hipStream_t s) {
  CM_CHECK_ARG(n_rows >= 0 && n_cols > 0 && x_row_stride >= n_cols);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(x && w && out && rstd && (!res || h));
  CM_CHECK_ARG(!low16 || (slot && small16 && n_small >= 0));  // n_small = 0: no tiny columns
  const int64_t blocks = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  const bool v8 = n_cols % 8 == 0 && x_row_stride % 8 == 0 && cm::aligned(x, 16) &&
                  cm::aligned(w, 16) && cm::aligned(out, 16) &&
                  (!low16 || cm::aligned(low16, 16)) &&
                  (!res || (cm::aligned(res, 16) && cm::aligned(h, 16)));
  const int vec = v8 ? 8 : 1;
  const int nv = pick_nv(n_cols, vec);
  // The output dtype is torch.promote_types(x, w), as in the reference (x: the norm's input,
  // fp32 h when a residual is added).
  CM_CHECK_ARG(out_dtype == promote(res ? static_cast<int>(CM_F32) : x_dtype, w_dtype));
  // rows of whole 512-column vectors and no tiny-|w| column to keep apart: one round trip a row
  const bool full = v8 && nv > 0 && n_cols % (cm::kWave * 8) == 0 && (!low16 || n_small == 0);
  if (res) {
    if (!full) {  // the add, then the general forward of h
      CM_CHECK_ARG(n_rows * n_cols / kThreads < 0x7fffffff);
      const unsigned g = static_cast<unsigned>((n_rows * n_cols + kThreads - 1) / kThreads);
      CM_FLOAT_SWITCH(x_dtype, XT, hipLaunchKernelGGL((residual_add_kernel<XT>), dim3(g),
                                                      dim3(kThreads), 0, s, res,
                                                      static_cast<const XT*>(x), x_row_stride,
                                                      h, n_rows, n_cols));
      return fwd_impl(h, CM_F32, n_cols, w, w_dtype, out, out_dtype, rstd, low16, slot, small16,
                      n_small, n_rows, n_cols, eps, nullptr, nullptr, s);
    }
    CM_FLOAT_SWITCH(x_dtype, XT, CM_FLOAT_SWITCH(w_dtype, WT, {
      CM_NV_SWITCH(nv, NV, if constexpr (NV > 0) hipLaunchKernelGGL(
                               (rmsnorm_fwd_full_kernel<XT, WT, float, NV, true>), dim3(blocks),
                               dim3(kThreads), 0, s, static_cast<const XT*>(x), x_row_stride,
                               static_cast<const WT*>(w), static_cast<float*>(out), rstd,
                               static_cast<_Float16*>(low16), res, h, n_rows, n_cols, eps));
    }));
    return cm::launch_status();
  }
  CM_FLOAT_SWITCH(x_dtype, XT, CM_FLOAT_SWITCH(w_dtype, WT, {
    using OT = Promoted<XT, WT>;
    if (full) {
      CM_NV_SWITCH(nv, NV, if constexpr (NV > 0) hipLaunchKernelGGL(
                               (rmsnorm_fwd_full_kernel<XT, WT, OT, NV, false>), dim3(blocks),
                               dim3(kThreads), 0, s, static_cast<const XT*>(x), x_row_stride,
                               static_cast<const WT*>(w), static_cast<OT*>(out), rstd,
                               static_cast<_Float16*>(low16), nullptr, nullptr, n_rows, n_cols,
                               eps));
    } else if (v8) {
      CM_NV_SWITCH(nv, NV, hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, WT, OT, 8, NV>),
                                              dim3(blocks), dim3(kThreads), 0, s,
                                              static_cast<const XT*>(x), x_row_stride,
                                              static_cast<const WT*>(w), static_cast<OT*>(out),
                                              rstd, static_cast<_Float16*>(low16), slot,
                                              static_cast<_Float16*>(small16), n_small, n_rows,
                                              n_cols, eps));
    } else {
      CM_NV_SWITCH(nv, NV, hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, WT, OT, 1, NV>),
                                              dim3(blocks), dim3(kThreads), 0, s,
                                              static_cast<const XT*>(x), x_row_stride,
                                              static_cast<const WT*>(w), static_cast<OT*>(out),
                                              rstd, static_cast<_Float16*>(low16), slot,
                                              static_cast<_Float16*>(small16), n_small, n_rows,
                                              n_cols, eps));
    }
  }));
  return cm::launch_status();
}

// cm_rmsnorm_bwd, and with `dres` / `dx16` cm_rmsnorm_bwd_res (fp32 x: dx = dres + the norm's
// dx, and its fp16 copy).
int bwd_impl(const void* dy, int dy_dtype, const void* xs, int xs_dtype, const void* w,
             int w_dtype, const float* rstd, void* dx, int dx_dtype, float* dw_partial,
             const int32_t* slot, const void* small16, int n_small, int saved_output,
             int64_t n_rows, int n_cols, const float* dres, void* dx16, hipStream_t s) {
  CM_CHECK_ARG(n_rows >= 0 && n_cols > 0);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(dy && xs && w && rstd && dx);
  const bool post = dres != nullptr || dx16 != nullptr;
  CM_CHECK_ARG(!post || dx_dtype == CM_F32);
  if (saved_output) {
    // xs holds the fp16 output copy; dx has the dtype of x (fp32 on this path); no dw.
    CM_CHECK_ARG(xs_dtype == CM_F16 && slot && small16 && n_small >= 0 && !dw_partial);
  }
  const bool want_dw = dw_partial != nullptr;
  const int64_t blocks = bwd_blocks(n_rows, want_dw);
  CM_CHECK_ARG(blocks <= 0x7fffffff);
  const bool v8 = n_cols % 8 == 0 && cm::aligned(dy, 16) && cm::aligned(xs, 16) &&
                  cm::aligned(w, 16) && cm::aligned(dx, 16) &&
                  (!dw_partial || cm::aligned(dw_partial, 16)) &&
                  (!dres || cm::aligned(dres, 16)) && (!dx16 || cm::aligned(dx16, 16));
  const int vec = v8 ? 8 : 1;
  const int nv = pick_nv(n_cols, vec);
  // The kernel's XT is the dtype of x (rounding target of gn/normed). On the saved-output path
  // x is fp32 and xs holds fp16 copies, read through the _Float16 view inside the kernel.
  const int x_dtype = saved_output ? dx_dtype : xs_dtype;
  // dx has the dtype of x; dy the dtype of the forward output, promote(x, w).
  CM_CHECK_ARG(dx_dtype == x_dtype && dy_dtype == promote(x_dtype, w_dtype));
  // rows of whole 512-column vectors, no tiny-|w| column map to read: the one-round-trip kernel
  const bool full = v8 && nv > 0 && n_cols % (cm::kWave * 8) == 0 && (!saved_output || n_small == 0);
  if (post && full) {  // fp32 x: one kernel
    CM_FLOAT_SWITCH(w_dtype, WT, {
      using DT = float;  // promote(fp32, w)
      if (saved_output) {
        CM_NV_SWITCH(nv, NV, if constexpr (NV > 0) hipLaunchKernelGGL(
                                 (rmsnorm_bwd_full_kernel<DT, float, WT, float, NV, true, true>),
                                 dim3(blocks), dim3(kThreads), 0, s, static_cast<const DT*>(dy),
                                 xs, static_cast<const WT*>(w), rstd, static_cast<float*>(dx),
                                 dw_partial, dres, static_cast<_Float16*>(dx16), n_rows,
                                 n_cols));
      } else {
        CM_NV_SWITCH(nv, NV, if constexpr (NV > 0) hipLaunchKernelGGL(
                                 (rmsnorm_bwd_full_kernel<DT, float, WT, float, NV, false, true>),
                                 dim3(blocks), dim3(kThreads), 0, s, static_cast<const DT*>(dy),
                                 xs, static_cast<const WT*>(w), rstd, static_cast<float*>(dx),
                                 dw_partial, dres, static_cast<_Float16*>(dx16), n_rows,
                                 n_cols));
      }
    });
    return cm::launch_status();
  }
  if (post) {  // the general backward, then the residual gradient over its dx
    const int rc = bwd_impl(dy, dy_dtype, xs, xs_dtype, w, w_dtype, rstd, dx, dx_dtype,
                            dw_partial, slot, small16, n_small, saved_output, n_rows, n_cols,
                            nullptr, nullptr, s);
    if (rc != 0) return rc;
    const int64_t n = n_rows * n_cols;
    CM_CHECK_ARG(n / kThreads < 0x7fffffff);
    hipLaunchKernelGGL(residual_grad_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, static_cast<float*>(dx), dres,
                       static_cast<_Float16*>(dx16), n);
    return cm::launch_status();
  }
  CM_FLOAT_SWITCH(x_dtype, XT, CM_FLOAT_SWITCH(w_dtype, WT, {
    using DT = Promoted<XT, WT>;
    using DXT = XT;
    if (full) {
      if (saved_output) {
        CM_NV_SWITCH(nv, NV, if constexpr (NV > 0) hipLaunchKernelGGL(
                                 (rmsnorm_bwd_full_kernel<DT, XT, WT, DXT, NV, true, false>),
                                 dim3(blocks), dim3(kThreads), 0, s, static_cast<const DT*>(dy),
                                 xs, static_cast<const WT*>(w), rstd, static_cast<DXT*>(dx),
                                 dw_partial, nullptr, nullptr, n_rows, n_cols));
      } else {
        CM_NV_SWITCH(nv, NV, if constexpr (NV > 0) hipLaunchKernelGGL(
                                 (rmsnorm_bwd_full_kernel<DT, XT, WT, DXT, NV, false, false>),
                                 dim3(blocks), dim3(kThreads), 0, s, static_cast<const DT*>(dy),
                                 xs, static_cast<const WT*>(w), rstd, static_cast<DXT*>(dx),
                                 dw_partial, nullptr, nullptr, n_rows, n_cols));
      }
    } else {
      if (v8) {
        CM_NV_SWITCH(nv, NV, hipLaunchKernelGGL((rmsnorm_bwd_kernel<DT, XT, WT, DXT, 8, NV>),
                                                dim3(blocks), dim3(kThreads), 0, s,
                                                static_cast<const DT*>(dy), xs,
                                                static_cast<const WT*>(w), rstd,
                                                static_cast<DXT*>(dx), dw_partial, slot,
                                                static_cast<const _Float16*>(small16), n_small,
                                                saved_output, n_rows, n_cols));
      } else {
        CM_NV_SWITCH(nv, NV, hipLaunchKernelGGL((rmsnorm_bwd_kernel<DT, XT, WT, DXT, 1, NV>),
                                                dim3(blocks), dim3(kThreads), 0, s,
                                                static_cast<const DT*>(dy), xs,
                                                static_cast<const WT*>(w), rstd,
                                                static_cast<DXT*>(dx), dw_partial, slot,
                                                static_cast<const _Float16*>(small16), n_small,
                                                saved_output, n_rows, n_cols));
      }
    }
  }));
  return cm::launch_status();
}

}  // namespace

extern "C" int cm_rmsnorm_fwd(const void* x, int x_dtype, int64_t x_row_stride, const void* w,
                              int w_dtype, void* out, int out_dtype, float* rstd, void* low16,
                              const int32_t* slot, void* small16, int n_small, int64_t n_rows,
                              int n_cols, float eps, void* stream) {
  return fwd_impl(x, x_dtype, x_row_stride, w, w_dtype, out, out_dtype, rstd, low16, slot,
                  small16, n_small, n_rows, n_cols, eps, nullptr, nullptr,
                  static_cast<hipStream_t>(stream));
}

extern "C" int cm_rmsnorm_add_fwd(const float* residual, const void* x, int x_dtype,
                                  int64_t x_row_stride, const void* w, int w_dtype, float* h,
                                  float* out, float* rstd, void* low16, const int32_t* slot,
                                  void* small16, int n_small, int64_t n_rows, int n_cols,
                                  float eps, void* stream) {
  CM_CHECK_ARG(n_rows == 0 || (residual != nullptr && h != nullptr));
  return fwd_impl(x, x_dtype, x_row_stride, w, w_dtype, out, CM_F32, rstd, low16, slot, small16,
                  n_small, n_rows, n_cols, eps, residual, h, static_cast<hipStream_t>(stream));
}

extern "C" int cm_rmsnorm_bwd(const void* dy, int dy_dtype, const void* xs, int xs_dtype,
                              const void* w, int w_dtype, const float* rstd, void* dx,
                              int dx_dtype, float* dw_partial, const int32_t* slot,
                              const void* small16, int n_small, int saved_output,
                              int64_t n_rows, int n_cols, void* stream) {
  return bwd_impl(dy, dy_dtype, xs, xs_dtype, w, w_dtype, rstd, dx, dx_dtype, dw_partial, slot,
                  small16, n_small, saved_output, n_rows, n_cols, nullptr, nullptr,
                  static_cast<hipStream_t>(stream));
}

extern "C" int cm_rmsnorm_bwd_res(const void* dy, int dy_dtype, const void* xs, int xs_dtype,
                                  const void* w, int w_dtype, const float* rstd,
                                  const float* dres, float* dx, void* dx16, float* dw_partial,
                                  const int32_t* slot, const void* small16, int n_small,
                                  int saved_output, int64_t n_rows, int n_cols, void* stream) {
  return bwd_impl(dy, dy_dtype, xs, xs_dtype, w, w_dtype, rstd, dx, CM_F32, dw_partial, slot,
                  small16, n_small, saved_output, n_rows, n_cols, dres, dx16,
                  static_cast<hipStream_t>(stream));
}
