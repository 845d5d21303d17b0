// INT8 symmetric per-output-channel weight quantisation for gfx950.
//
// Bit-exact restatement of the reference's weight path:
//   scale[n] = max(max_k |W[n,k]|, 1e-8) / 127        (cortex/quantization/calibrate.py:154)
//   q[n,k]   = clamp(rint(W[n,k] / scale[n]), -127, 127)  (calibrate.py:216-220)
// Division and the 1/127 step are IEEE fp32 divisions (hipcc rounds fp32 '/'
// correctly by default); rint rounds half to even like Tensor.round().
#include <hip/hip_runtime.h>

#include "common.h"

namespace cortex {

// one wavefront per output channel
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ w, int64_t N, int64_t K,
                                                             int64_t ld_w, const float* __restrict__ scale_in,
                                                             float* __restrict__ scale_out, int8_t* __restrict__ q,
                                                             int64_t ld_q) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (n >= N) return;
  const float* row = w + n * ld_w;
  float s;
  if (scale_in) {
    s = scale_in[n];
  } else {
    float amax = 0.0f;
    for (int64_t k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(row[k]));
    amax = wave_max(amax);
    s = fmaxf(amax, 1e-8f) / 127.0f;
  }
  if (scale_out && lane == 0) scale_out[n] = s;
  if (q == nullptr) return;  // scale-only request
  int8_t* qr = q + n * ld_q;
  for (int64_t k = lane; k < K; k += 64) {
    float v = rintf(row[k] / s);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    qr[k] = (int8_t)(int)v;
  }
}

}  // namespace cortex

using namespace cortex;

extern "C" int cortex_quantize_int8(const float* w, int64_t N, int64_t K, int64_t ld_w, const float* scale_in,
                                    float* scale_out, int8_t* q, int64_t ld_q, hipStream_t stream) {
  CORTEX_CHECK_ARG(N >= 0 && K >= 0, "cortex_quantize_int8: negative shape");
  if (N == 0) return OK;
  CORTEX_CHECK_ARG(w && (q || scale_out), "cortex_quantize_int8: null weight, or neither q nor scale_out");
  CORTEX_CHECK_ARG(ld_w >= K && ld_q >= K, "cortex_quantize_int8: row strides must be >= K");
  CORTEX_CHECK_ARG(scale_in || scale_out, "cortex_quantize_int8: need scale_in or scale_out");
  const int rows_per_block = 4;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)cdiv(N, rows_per_block)), dim3(256), 0, stream, w, N, K,
                     ld_w, scale_in, scale_out, q, ld_q);
  CORTEX_CHECK_LAUNCH("quantize_rows_kernel");
  return OK;
}
