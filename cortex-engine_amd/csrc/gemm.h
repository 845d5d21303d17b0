// Arguments shared by the general and the tiled GEMM kernels.
#pragma once

#include "common.h"

namespace cortex {

enum NormMode : int { NORM_NONE = 0, NORM_LAYER = 1, NORM_RMS = 2 };
enum ActMode : int { ACT_NONE = 0, ACT_GELU = 1 };

struct GemmArgs {
  int64_t M, N, K;
  const void* x;
  int64_t ld_x;
  int norm;
  const float2* stats;
  const void* gamma;
  const void* beta;
  int gamma_dtype;
  const void* w;
  int64_t ld_w;
  const float* w_scale;
  const void* bias;
  int bias_dtype;
  int act;
  const void* res;
  int res_dtype;
  int64_t ld_res;
  int64_t res_rows;
  void* out;
  int out_dtype;
  int64_t ld_out;
  int vec;  // 1: 16-byte aligned rows, vector loads allowed
  // int8 x int8 kernels only (gemm_bf16.hip, TIN = int8_t): x holds round(x_f / a_scale),
  // and an int8 output is written as clamp(rint(y * out_inv_scale), -127, 127)
  float a_scale;
  float out_inv_scale;
  // bf16 row-scaled kernels only (gemm_bf16.hip, RS): the accumulator of row m is scaled by
  // 1 / sqrt(mean_k(x[m, k]^2) + rms_eps) before the weight scale (RMSNorm without a gain)
  float rms_eps;
};

// bf16 x bf16 path with a register epilogue (gemm_bf16.hip), same return convention.
int try_gemm_bf16(const GemmArgs& g, int x_dtype, int w_dtype, int w_layout, int compute, hipStream_t stream);

// The direct-weight residual GEMM (gemm_bf16.hip): bf16 x, w in MFMA fragment order
// (DT_BF16_FRAG), fp32 residual and output, N % 128 == 0, K 1024 / 2048 / 3072, 16-byte
// aligned rows.  Returns OK or an error status.
int launch_res_dw(const GemmArgs& g, hipStream_t stream);

// K split over gridDim.z = splits workgroup slabs (gemm_bf16.hip): slab z computes
// (x[:, zK:(z+1)K] . w[:, zK:(z+1)K]^T) * w_scale into g.out + z * M * ld_out (fp32), where
// K = g.K is the per-slab depth (a multiple of 64) and g.x / g.w are the full rows.  No
// bias, activation or residual.  Returns 1 when launched, 0 when the grid is too large.
int split_k_partials(const GemmArgs& g, int splits, hipStream_t stream);

}  // namespace cortex
