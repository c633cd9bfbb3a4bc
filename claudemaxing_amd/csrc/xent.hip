// Cross-entropy statistics of full logits rows (gfx950): the fallback used when the logits
// exist anyway. Reproduces solution/lm_head_loss.py:54-96 (lm_head_xent_rows_kernel):
//   per row: M = max z, S = sum e^{z-M}, D = sum e^{z-M} z, lse = M + ln S,
//   loss = label ? lse - z[t] : 0, entropy = lse - D/S, correct = label && argmax == t
//   (first index of the maximum), and optionally the row overwritten by
//   round((softmax - onehot) * grad_scale), zero for unlabelled rows.
//
// One 256-lane workgroup per row; each lane keeps an online (max, sum, dot, argmax) state over
// its columns, then the states are merged across the wavefront with shuffles and across the
// four wavefronts through LDS. e^x is computed as 2^(x log2 e) on v_exp_f32, ln as
// log2 * ln 2 on v_log_f32.
#include "common.h"

#include "softmax_state.h"

namespace {

constexpr int kThreads = 256;

template <typename T>
__global__ __launch_bounds__(kThreads) void xent_rows_kernel(T* __restrict__ logits,
                                                             int64_t row_stride,
                                                             const int64_t* __restrict__ target,
                                                             float* __restrict__ loss,
                                                             float* __restrict__ entropy,
                                                             int32_t* __restrict__ correct,
                                                             int64_t n_cols, int write_grad,
                                                             float grad_scale) {
  const int64_t row = blockIdx.x;
  T* z = logits + row * row_stride;
  cm::SoftmaxState st = cm::SoftmaxState::empty();
  for (int64_t c = threadIdx.x; c < n_cols; c += kThreads) st.push(cm::to_f32(z[c]), c);
  __shared__ cm::SoftmaxState s_part[kThreads / cm::kWave];
  st = cm::block_merge<kThreads>(st, s_part);
  const int64_t t = target[row];
  const bool labelled = t != -100;
  // A label outside [0, n_cols) is not read: its loss is NaN.
  const bool in_range = t >= 0 && t < n_cols;
  const float lse = st.lse();
  if (threadIdx.x == 0) {
    const float zt = in_range ? cm::to_f32(z[t]) : __builtin_nanf("");
    loss[row] = labelled ? lse - zt : 0.0f;
    entropy[row] = lse - st.dot / st.sum;
    correct[row] = labelled && st.best == t ? 1 : 0;
  }
  if (write_grad) {
    __syncthreads();  // every lane has read its logits (and z[t]) before any is overwritten
    for (int64_t c = threadIdx.x; c < n_cols; c += kThreads) {
      float g = 0.0f;
      if (labelled) {
        const float p = cm::exp_f(cm::to_f32(z[c]) - lse);
        g = (c == t ? p - 1.0f : p) * grad_scale;
      }
      z[c] = cm::from_f32<T>(g);
    }
  }
}

}  // namespace

extern "C" int cm_xent_rows(void* logits, int logits_dtype, int64_t row_stride,
                            const int64_t* target, float* loss, float* entropy, int32_t* correct,
                            int64_t n_rows, int64_t n_cols, int write_grad, float grad_scale,
                            void* stream) {
  CM_CHECK_ARG(n_rows >= 0 && n_cols > 0 && row_stride >= n_cols);
  if (n_rows == 0) return 0;
  CM_CHECK_ARG(logits && target && loss && entropy && correct);
  CM_CHECK_ARG(n_rows <= 0x7fffffff);
  hipStream_t s = static_cast<hipStream_t>(stream);
  CM_FLOAT_SWITCH(logits_dtype, T, {
    hipLaunchKernelGGL((xent_rows_kernel<T>), dim3(static_cast<uint32_t>(n_rows)),
                       dim3(kThreads), 0, s, static_cast<T*>(logits), row_stride, target, loss,
                       entropy, correct, n_cols, write_grad, grad_scale);
  });
  return cm::launch_status();
}
