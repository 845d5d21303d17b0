// Row-wise helpers for the Cortex forward on gfx950.
//
//   cortex_convert       elementwise dtype conversion (int8 / f32 / bf16 / f16 -> f32 / bf16),
//                        used to build the bf16 execution image of INT8 weights (exact)
//                        and fp32 copies of small parameter vectors;
//   cortex_ln_rows       LayerNorm of rows with K = 64 * EPL held in registers (one
//                        wavefront per row, two-pass mean/variance), optionally a second
//                        LayerNorm applied to the result (the encoder's final_norm feeding
//                        the behaviour head's norm), written as bf16 and/or fp32.
#include <hip/hip_runtime.h>

#include "common.h"

namespace cortex {

template <class TI, class TO>
__global__ __launch_bounds__(256) void convert_kernel(const TI* __restrict__ in, TO* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = from_f32<TO>(to_f32(in[i]));
}

// One LayerNorm pass over the EPL values a lane holds (row spread over the wave).
template <int EPL>
__device__ __forceinline__ void ln_regs(float (&v)[EPL], float inv_k, float eps, const float* __restrict__ gamma,
                                        const float* __restrict__ beta, int lane) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) s += v[j];
  const float mean = wave_sum(s) * inv_k;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const float d = v[j] - mean;
    ss += d * d;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) * inv_k + eps);
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    // element k = (j / 4) * 256 + lane * 4 + (j % 4)
    const int k = (j >> 2) * 256 + lane * 4;
    const float4 gm = gamma ? *reinterpret_cast<const float4*>(gamma + k) : make_float4(1.f, 1.f, 1.f, 1.f);
    const float4 bt = beta ? *reinterpret_cast<const float4*>(beta + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    v[j] = (v[j] - mean) * rstd * gm.x + bt.x;
    v[j + 1] = (v[j + 1] - mean) * rstd * gm.y + bt.y;
    v[j + 2] = (v[j + 2] - mean) * rstd * gm.z + bt.z;
    v[j + 3] = (v[j + 3] - mean) * rstd * gm.w + bt.w;
  }
}

// Row r: lane l holds elements (j/4)*256 + 4l + (j%4), loaded as float4 (coalesced).
template <int EPL>
__global__ __launch_bounds__(256) void ln_rows_kernel(const float* __restrict__ x, int64_t M, int64_t ld_x,
                                                       const float* g1, const float* b1, float eps1,
                                                       const float* g2, const float* b2, float eps2, int two,
                                                       bf16* __restrict__ out_bf, int64_t ld_bf,
                                                       float* __restrict__ out_f, int64_t ld_f) {
  constexpr int K = 64 * EPL;
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (m >= M) return;
  const float* row = x + m * ld_x;
  float v[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    const float4 q = *reinterpret_cast<const float4*>(row + (j >> 2) * 256 + lane * 4);
    v[j] = q.x;
    v[j + 1] = q.y;
    v[j + 2] = q.z;
    v[j + 3] = q.w;
  }
  const float inv_k = 1.0f / (float)K;
  ln_regs<EPL>(v, inv_k, eps1, g1, b1, lane);
  if (two) ln_regs<EPL>(v, inv_k, eps2, g2, b2, lane);
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    const int k = (j >> 2) * 256 + lane * 4;
    if (out_bf) {
      bf16x4 b;
      b[0] = (bf16)v[j];
      b[1] = (bf16)v[j + 1];
      b[2] = (bf16)v[j + 2];
      b[3] = (bf16)v[j + 3];
      *reinterpret_cast<bf16x4*>(out_bf + m * ld_bf + k) = b;
    }
    if (out_f) *reinterpret_cast<float4*>(out_f + m * ld_f + k) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
  }
}

}  // namespace cortex

using namespace cortex;

extern "C" {

int cortex_convert(int in_dtype, const void* in, int out_dtype, void* out, int64_t n, hipStream_t stream) {
  CORTEX_CHECK_ARG(n >= 0, "cortex_convert: negative length");
  if (n == 0) return OK;
  CORTEX_CHECK_ARG(in && out, "cortex_convert: null pointer");
  const dim3 grid((unsigned)std::min<int64_t>(cdiv(n, 256), 4096));
#define CORTEX_CVT(TI, TO) \
  hipLaunchKernelGGL((convert_kernel<TI, TO>), grid, dim3(256), 0, stream, (const TI*)in, (TO*)out, n)
  if (out_dtype == DT_BF16) {
    if (in_dtype == DT_I8) CORTEX_CVT(int8_t, bf16);
    else if (in_dtype == DT_F32) CORTEX_CVT(float, bf16);
    else if (in_dtype == DT_BF16) CORTEX_CVT(bf16, bf16);
    else if (in_dtype == DT_F16) CORTEX_CVT(f16, bf16);
    else { set_error("cortex_convert: unsupported input dtype %d", in_dtype); return E_UNSUPPORTED; }
  } else if (out_dtype == DT_F32) {
    if (in_dtype == DT_I8) CORTEX_CVT(int8_t, float);
    else if (in_dtype == DT_F32) CORTEX_CVT(float, float);
    else if (in_dtype == DT_BF16) CORTEX_CVT(bf16, float);
    else if (in_dtype == DT_F16) CORTEX_CVT(f16, float);
    else { set_error("cortex_convert: unsupported input dtype %d", in_dtype); return E_UNSUPPORTED; }
  } else {
    set_error("cortex_convert: unsupported output dtype %d", out_dtype);
    return E_UNSUPPORTED;
  }
#undef CORTEX_CVT
  CORTEX_CHECK_LAUNCH("convert_kernel");
  return OK;
}

int cortex_ln_rows(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma1, const float* beta1,
                   float eps1, const float* gamma2, const float* beta2, float eps2, void* out_bf16, int64_t ld_bf16,
                   float* out_f32, int64_t ld_f32, hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0, "cortex_ln_rows: negative M");
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(x && (out_bf16 || out_f32), "cortex_ln_rows: null input or no output");
  CORTEX_CHECK_ARG(K == 256 || K == 512 || K == 768 || K == 1024,
                   "cortex_ln_rows: K=%lld not one of 256, 512, 768, 1024", (long long)K);
  CORTEX_CHECK_ARG(((uintptr_t)x & 15) == 0 && ld_x % 4 == 0, "cortex_ln_rows: x rows must be 16-byte aligned");
  CORTEX_CHECK_ARG(!out_bf16 || (((uintptr_t)out_bf16 & 7) == 0 && ld_bf16 % 4 == 0),
                   "cortex_ln_rows: bf16 output rows must be 8-byte aligned");
  CORTEX_CHECK_ARG(!out_f32 || (((uintptr_t)out_f32 & 15) == 0 && ld_f32 % 4 == 0),
                   "cortex_ln_rows: fp32 output rows must be 16-byte aligned");
  for (const float* p : {gamma1, beta1, gamma2, beta2})
    CORTEX_CHECK_ARG(((uintptr_t)p & 15) == 0, "cortex_ln_rows: gamma/beta must be 16-byte aligned fp32");
  const int two = gamma2 != nullptr || beta2 != nullptr;
  const dim3 grid((unsigned)cdiv(M, 4));
#define CORTEX_LNR(EPL)                                                                                          \
  hipLaunchKernelGGL((ln_rows_kernel<EPL>), grid, dim3(256), 0, stream, x, M, ld_x, gamma1, beta1, eps1, gamma2, \
                     beta2, eps2, two, (bf16*)out_bf16, ld_bf16, out_f32, ld_f32)
  switch (K) {
    case 256: CORTEX_LNR(4); break;
    case 512: CORTEX_LNR(8); break;
    case 768: CORTEX_LNR(12); break;
    default: CORTEX_LNR(16); break;
  }
#undef CORTEX_LNR
  CORTEX_CHECK_LAUNCH("ln_rows_kernel");
  return OK;
}

}  // extern "C"
