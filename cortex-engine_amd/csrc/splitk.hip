// Residual linears with K split across workgroups, for small row counts.
//
// At batch 1 the residual linears of a Perceiver block have M = 256 rows: the
// MLP-down GEMM (K = 2048) covers 8 column tiles and the out-projection + LayerNorm
// kernel 8 row blocks, i.e. 8 CUs, each walking the whole K.  Here K is cut into
// `splits` slabs: slab z of every output tile is its own workgroup (gemm_bf16.hip's
// kernel on grid z) and writes the scaled partial product to its fp32 slab of the
// caller's workspace; a second kernel sums the slabs in slab order (fixed, so results
// repeat bit for bit) and adds bias and residual -- and, for the LayerNorm variant,
// writes the LayerNorm of the new rows as bf16, one wavefront per row.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "gemm.h"

namespace cortex {

namespace {

struct ReduceArgs {
  const float* part;  // (splits, M, N) slabs
  int64_t splits, M, N;
  const float* bias;  // (N) or null
  const float* res;   // row m % res_rows, stride ld_res
  int64_t ld_res, res_rows;
  float* out;
  int64_t ld_out;
};

__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs a) {
  const int64_t groups = a.M * (a.N >> 2);
  const WtOut store(a.out, a.M * a.ld_out * 4, true);  // few rows (the K split serves B <= 8)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < groups; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / (a.N >> 2), c = (i - m * (a.N >> 2)) * 4;
    const float* p = a.part + m * a.N + c;
    float4 s = *reinterpret_cast<const float4*>(p);
    for (int64_t z = 1; z < a.splits; ++z) {
      const float4 t = *reinterpret_cast<const float4*>(p + z * a.M * a.N);
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    if (a.bias) {
      const float4 b = *reinterpret_cast<const float4*>(a.bias + c);
      s.x += b.x; s.y += b.y; s.z += b.z; s.w += b.w;
    }
    const float4 r = *reinterpret_cast<const float4*>(a.res + (m % a.res_rows) * a.ld_res + c);
    store(reinterpret_cast<float4*>(a.out + m * a.ld_out + c), make_float4(s.x + r.x, s.y + r.y, s.z + r.z, s.w + r.w));
  }
}

struct ReduceLnArgs {
  ReduceArgs r;
  const float* gamma;
  const float* beta;
  float eps;
  bf16* xn;
  int64_t ld_xn;
};

// one wavefront per row; lane holds elements (j / 4) * 256 + 4 lane + j % 4
template <int EPL>
__global__ __launch_bounds__(256) void splitk_reduce_ln_kernel(ReduceLnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (m >= a.r.M) return;
  const int64_t N = a.r.N;
  const WtOut store_x(a.r.out, a.r.M * a.r.ld_out * 4, true), store_xn(a.xn, a.r.M * a.ld_xn * 2, true);
  float v[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    const int k = (j >> 2) * 256 + lane * 4;
    const float* p = a.r.part + m * N + k;
    float4 s = *reinterpret_cast<const float4*>(p);
    for (int64_t z = 1; z < a.r.splits; ++z) {
      const float4 t = *reinterpret_cast<const float4*>(p + z * a.r.M * N);
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    if (a.r.bias) {
      const float4 b = *reinterpret_cast<const float4*>(a.r.bias + k);
      s.x += b.x; s.y += b.y; s.z += b.z; s.w += b.w;
    }
    const float4 r = *reinterpret_cast<const float4*>(a.r.res + (m % a.r.res_rows) * a.r.ld_res + k);
    v[j] = s.x + r.x;
    v[j + 1] = s.y + r.y;
    v[j + 2] = s.z + r.z;
    v[j + 3] = s.w + r.w;
    store_x(reinterpret_cast<float4*>(a.r.out + m * a.r.ld_out + k), make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]));
  }
  ln_regs<EPL>(v, 1.0f / (float)N, a.eps, a.gamma, a.beta, lane);
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    bf16x4 o;
    o[0] = (bf16)v[j];
    o[1] = (bf16)v[j + 1];
    o[2] = (bf16)v[j + 2];
    o[3] = (bf16)v[j + 3];
    store_xn(reinterpret_cast<bf16x4*>(a.xn + m * a.ld_xn + (j >> 2) * 256 + lane * 4), o);
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// validate the shared operands and launch the partial products into the workspace
int partials(const char* who, int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, const void* w,
             int64_t ld_w, const float* w_scale, const float* bias, const float* res, int64_t ld_res,
             int64_t res_rows, const float* out, int64_t ld_out, int64_t splits, void* workspace,
             int64_t workspace_bytes, hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 1 && N >= 8 && N % 8 == 0, "%s: need M >= 1 and N a positive multiple of 8", who);
  CORTEX_CHECK_ARG(splits >= 1 && splits <= 64 && K > 0 && K % (64 * splits) == 0,
                   "%s: K must be a positive multiple of 64 * splits (splits in [1, 64])", who);
  CORTEX_CHECK_ARG(M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= 0x7fffffffLL, "%s: size too large", who);
  CORTEX_CHECK_ARG(x && w && res && out, "%s: null pointer", who);
  CORTEX_CHECK_ARG(res_rows >= 0 && ld_x >= K && ld_w >= K && ld_res >= N && ld_out >= N, "%s: row strides too small",
                   who);
  CORTEX_CHECK_ARG(al16(x) && al16(w) && ld_x % 8 == 0 && ld_w % 8 == 0 && al16(res) && al16(out) && ld_res % 4 == 0 &&
                       ld_out % 4 == 0 && (!w_scale || al16(w_scale)) && (!bias || al16(bias)),
                   "%s: operands must be 16-byte aligned rows", who);
  const int64_t need = splits * M * N * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need || !al16(workspace)) {
    set_error("%s: workspace of %lld bytes (16-byte aligned) is smaller than the required %lld", who,
              (long long)workspace_bytes, (long long)need);
    return E_WORKSPACE;
  }
  GemmArgs g = {};
  g.M = M;
  g.N = N;
  g.K = K / splits;
  g.x = x;
  g.ld_x = ld_x;
  g.w = w;
  g.ld_w = ld_w;
  g.w_scale = w_scale;
  g.bias_dtype = DT_F32;
  g.out = workspace;
  g.out_dtype = DT_F32;
  g.ld_out = N;
  g.vec = 1;
  if (split_k_partials(g, (int)splits, stream) != 1) {
    set_error("%s: grid too large", who);
    return E_INVALID;
  }
  return OK;
}

}  // namespace

}  // namespace cortex

using namespace cortex;

extern "C" int64_t cortex_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits) {
  if (M <= 0 || N <= 0 || splits <= 0) return 0;
  return splits * M * N * (int64_t)sizeof(float);
}

extern "C" int cortex_linear_residual_splitk(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x,
                                             const void* w, int64_t ld_w, const float* w_scale, const float* bias,
                                             const float* res, int64_t ld_res, int64_t res_rows, float* out,
                                             int64_t ld_out, int64_t splits, void* workspace,
                                             int64_t workspace_bytes, hipStream_t stream) {
  const char* who = "cortex_linear_residual_splitk";
  if (M == 0) return OK;
  const int st = partials(who, M, N, K, x, ld_x, w, ld_w, w_scale, bias, res, ld_res, res_rows, out, ld_out, splits,
                          workspace, workspace_bytes, stream);
  if (st != OK) return st;
  ReduceArgs a{reinterpret_cast<const float*>(workspace), splits, M, N, bias, res, ld_res, res_rows > 0 ? res_rows : M,
               out, ld_out};
  const int64_t groups = M * (N / 4);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)std::min<int64_t>(cdiv(groups, 256), 4096)), dim3(256), 0,
                     stream, a);
  CORTEX_CHECK_LAUNCH("splitk_reduce_kernel");
  return OK;
}

extern "C" int cortex_linear_residual_ln_splitk(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x,
                                                const void* w, int64_t ld_w, const float* w_scale, const float* bias,
                                                const float* res, int64_t ld_res, int64_t res_rows, float* out,
                                                int64_t ld_out, const float* gamma, const float* beta, float eps,
                                                void* xn, int64_t ld_xn, int64_t splits, void* workspace,
                                                int64_t workspace_bytes, hipStream_t stream) {
  const char* who = "cortex_linear_residual_ln_splitk";
  CORTEX_CHECK_ARG(N == 256 || N == 512 || N == 768 || N == 1024, "%s: N must be 256, 512, 768 or 1024", who);
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(gamma && beta && xn && al16(gamma) && al16(beta) && ((uintptr_t)xn & 7) == 0 && ld_xn >= N &&
                       ld_xn % 4 == 0,
                   "%s: LayerNorm parameters and xn rows must be aligned", who);
  const int st = partials(who, M, N, K, x, ld_x, w, ld_w, w_scale, bias, res, ld_res, res_rows, out, ld_out, splits,
                          workspace, workspace_bytes, stream);
  if (st != OK) return st;
  ReduceLnArgs a{{reinterpret_cast<const float*>(workspace), splits, M, N, bias, res, ld_res,
                  res_rows > 0 ? res_rows : M, out, ld_out},
                 gamma, beta, eps, reinterpret_cast<bf16*>(xn), ld_xn};
  const dim3 grid((unsigned)cdiv(M, 4));
  switch (N) {
    case 256: hipLaunchKernelGGL(splitk_reduce_ln_kernel<4>, grid, dim3(256), 0, stream, a); break;
    case 512: hipLaunchKernelGGL(splitk_reduce_ln_kernel<8>, grid, dim3(256), 0, stream, a); break;
    case 768: hipLaunchKernelGGL(splitk_reduce_ln_kernel<12>, grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(splitk_reduce_ln_kernel<16>, grid, dim3(256), 0, stream, a); break;
  }
  CORTEX_CHECK_LAUNCH("splitk_reduce_ln_kernel");
  return OK;
}
