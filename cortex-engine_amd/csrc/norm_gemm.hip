// Fused row-norm + linear for gfx950:  y = epi( norm(x) . W^T )
//
//   norm   none | LayerNorm (x-mean)*rstd*gamma+beta | RMSNorm (x/rms)*gamma, applied
//          to the A tile while it is staged into LDS; the per-row statistics come
//          from row_stats_kernel (one wavefront per row, two-pass mean/variance).
//          The normalised row is rounded to the compute dtype before the
//          contraction, as the reference does with x_norm.to(x.dtype)
//          (cortex/kernels/fused_rmsnorm.py:100-106).
//   W      int8 (N, K) row-major with a per-row fp32 scale (QuantizedLinear's
//          weight_int8/weight_scale, cortex/quantization/calibrate.py:192-193),
//          widened exactly to bf16/fp32 in LDS; or bf16/fp32 (N, K) or (K, N).
//   MFMA   bf16 compute: v_mfma_f32_16x16x32_bf16; fp32 compute: v_mfma_f32_16x16x4_f32,
//          fp32 accumulation in both.
//   epi    y = acc * scale[n] (+ bias[n]) (-> GELU) (+ residual[m % res_rows, n]).
//
// Tiling: 256 threads = 4 wavefronts in a 2x2 grid, 128x128 output tile per
// workgroup, 64x64 per wavefront (4x4 MFMA tiles), BK = 64 (bf16) / 32 (fp32),
// two LDS stages with register prefetch of the next K tile.
#include <hip/hip_runtime.h>

#include "common.h"
#include "gemm.h"

namespace cortex {

__device__ __forceinline__ float load_f32(const void* p, int dtype, int64_t i) {
  if (dtype == DT_BF16) return (float)reinterpret_cast<const bf16*>(p)[i];
  if (dtype == DT_F16) return (float)reinterpret_cast<const f16*>(p)[i];
  return reinterpret_cast<const float*>(p)[i];
}
__device__ __forceinline__ void store_f32(void* p, int dtype, int64_t i, float v) {
  if (dtype == DT_BF16)
    reinterpret_cast<bf16*>(p)[i] = (bf16)v;
  else if (dtype == DT_F16)
    reinterpret_cast<f16*>(p)[i] = (f16)v;
  else
    reinterpret_cast<float*>(p)[i] = v;
}

// --------------------------------------------------------------------------
// Row statistics: LN -> (mean, rstd); RMS -> (0, rms).  One wavefront per row.
// --------------------------------------------------------------------------
template <class TX>
__global__ __launch_bounds__(256) void row_stats_kernel(const TX* __restrict__ x, int64_t M, int64_t K, int64_t ld,
                                                         int norm, float eps, float2* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (m >= M) return;
  const TX* row = x + m * ld;
  const float inv_k = 1.0f / (float)K;
  if (norm == NORM_RMS) {
    float ss = 0.0f;
    for (int64_t k = lane; k < K; k += 64) {
      const float v = to_f32(row[k]);
      ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) stats[m] = make_float2(0.0f, sqrtf(ss * inv_k + eps));
  } else {
    float s = 0.0f;
    for (int64_t k = lane; k < K; k += 64) s += to_f32(row[k]);
    const float mean = wave_sum(s) * inv_k;
    float ss = 0.0f;
    for (int64_t k = lane; k < K; k += 64) {
      const float d = to_f32(row[k]) - mean;
      ss += d * d;
    }
    const float var = wave_sum(ss) * inv_k;
    if (lane == 0) stats[m] = make_float2(mean, 1.0f / sqrtf(var + eps));
  }
}

// LayerNorm applied and written out: y = (x - mean) * rstd * gamma + beta.
template <class TX, class TY>
__global__ __launch_bounds__(256) void layer_norm_kernel(const TX* __restrict__ x, int64_t M, int64_t K, int64_t ld,
                                                          const void* gamma, const void* beta, int gdt, float eps,
                                                          TY* __restrict__ y, int64_t ld_y) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (m >= M) return;
  const TX* row = x + m * ld;
  const float inv_k = 1.0f / (float)K;
  float s = 0.0f;
  for (int64_t k = lane; k < K; k += 64) s += to_f32(row[k]);
  const float mean = wave_sum(s) * inv_k;
  float ss = 0.0f;
  for (int64_t k = lane; k < K; k += 64) {
    const float d = to_f32(row[k]) - mean;
    ss += d * d;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) * inv_k + eps);
  TY* out = y + m * ld_y;
  for (int64_t k = lane; k < K; k += 64) {
    const float gm = gamma ? load_f32(gamma, gdt, k) : 1.0f;
    const float bt = beta ? load_f32(beta, gdt, k) : 0.0f;
    out[k] = from_f32<TY>((to_f32(row[k]) - mean) * rstd * gm + bt);
  }
}

// --------------------------------------------------------------------------
// GEMM
// --------------------------------------------------------------------------


template <class TC>
struct TileCfg;
template <>
struct TileCfg<bf16> {
  static constexpr int BK = 64, PAD = 8;
};
template <>
struct TileCfg<float> {
  static constexpr int BK = 32, PAD = 4;
};

constexpr int GEMM_BM = 128, GEMM_BN = 128, GEMM_THREADS = 256;

// 8 consecutive source elements held in registers between the global load and the
// LDS store (kept raw so that the loads stay in flight across the MFMA phase).
template <class T>
struct Raw8 {
  T v[8];
};

template <class T>
__device__ __forceinline__ void load8(Raw8<T>& r, const T* p, bool full, int valid, bool vec) {
  if (full && vec) {
    if constexpr (sizeof(T) == 1) {
      *reinterpret_cast<uint2*>(r.v) = *reinterpret_cast<const uint2*>(p);
    } else if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(r.v) = *reinterpret_cast<const uint4*>(p);
    } else {
      reinterpret_cast<uint4*>(r.v)[0] = reinterpret_cast<const uint4*>(p)[0];
      reinterpret_cast<uint4*>(r.v)[1] = reinterpret_cast<const uint4*>(p)[1];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) r.v[j] = (j < valid) ? p[j] : T(0);
  }
}

template <class TC>
__device__ __forceinline__ void store8_lds(TC* dst, const float (&f)[8]) {
  if constexpr (sizeof(TC) == 2) {
    bf16x8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (bf16)f[j];
    *reinterpret_cast<bf16x8*>(dst) = v;
  } else {
    f32x4 a = {f[0], f[1], f[2], f[3]}, b = {f[4], f[5], f[6], f[7]};
    reinterpret_cast<f32x4*>(dst)[0] = a;
    reinterpret_cast<f32x4*>(dst)[1] = b;
  }
}

template <class TC>
__device__ __forceinline__ Frag<TC> lds_frag(const TC* p) {
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    const f32x4 a = reinterpret_cast<const f32x4*>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4*>(p)[1];
    f.v = (f32x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
  return f;
}

template <class TX, class TC, class TW, bool W_KN>
__global__ __launch_bounds__(GEMM_THREADS, 2) void gemm_kernel(GemmArgs g) {
  constexpr int BM = GEMM_BM, BN = GEMM_BN, BK = TileCfg<TC>::BK, LDK = BK + TileCfg<TC>::PAD;
  constexpr int CH_A = BM * BK / 8 / GEMM_THREADS;  // 8-element chunks per thread
  constexpr int CH_B = BN * BK / 8 / GEMM_THREADS;
  constexpr int KCH = BK / 8;  // chunks per tile row
  __shared__ __attribute__((aligned(16))) TC As[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) TC Bs[2][BN][LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int64_t M = g.M, N = g.N, K = g.K;
  const TX* __restrict__ X = reinterpret_cast<const TX*>(g.x);
  const TW* __restrict__ W = reinterpret_cast<const TW*>(g.w);
  const bool vec = g.vec != 0;

  // per-thread row statistics for the A rows it stages (constant over K)
  float st_a[CH_A], st_b[CH_A];
#pragma unroll
  for (int c = 0; c < CH_A; ++c) {
    const int ci = tid + c * GEMM_THREADS;
    const int64_t m = m0 + ci / KCH;
    float2 s = make_float2(0.0f, 1.0f);
    if (g.norm != NORM_NONE && m < M) s = g.stats[m];
    st_a[c] = s.x;
    st_b[c] = s.y;
  }

  Raw8<TX> ra[CH_A];
  Raw8<TW> rb[CH_B];

  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < CH_A; ++c) {
      const int ci = tid + c * GEMM_THREADS;
      const int64_t m = m0 + ci / KCH;
      const int64_t k = k0 + (ci % KCH) * 8;
      const int valid = (m < M) ? (int)max<int64_t>(0, min<int64_t>(8, K - k)) : 0;
      load8(ra[c], X + (m < M ? m : 0) * g.ld_x + (valid > 0 ? k : 0), valid == 8, valid, vec);
    }
#pragma unroll
    for (int c = 0; c < CH_B; ++c) {
      const int ci = tid + c * GEMM_THREADS;
      if (!W_KN) {
        const int64_t n = n0 + ci / KCH;
        const int64_t k = k0 + (ci % KCH) * 8;
        const int valid = (n < N) ? (int)max<int64_t>(0, min<int64_t>(8, K - k)) : 0;
        load8(rb[c], W + (n < N ? n : 0) * g.ld_w + (valid > 0 ? k : 0), valid == 8, valid, vec);
      } else {
        // (K, N) layout: chunk = 8 consecutive n at one k
        constexpr int NCH = BN / 8;
        const int64_t k = k0 + ci / NCH;
        const int64_t n = n0 + (ci % NCH) * 8;
        const int valid = (k < K) ? (int)max<int64_t>(0, min<int64_t>(8, N - n)) : 0;
        load8(rb[c], W + (k < K ? k : 0) * g.ld_w + (valid > 0 ? n : 0), valid == 8, valid, vec);
      }
    }
  };

  auto store_tiles = [&](int buf, int64_t k0) {
#pragma unroll
    for (int c = 0; c < CH_A; ++c) {
      const int ci = tid + c * GEMM_THREADS;
      const int r = ci / KCH, kc = (ci % KCH) * 8;
      float f[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = to_f32(ra[c].v[j]);
      if (g.norm != NORM_NONE) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t k = k0 + kc + j;
          if (k < K) {
            const float gm = load_f32(g.gamma, g.gamma_dtype, k);
            if (g.norm == NORM_LAYER) {
              const float bt = g.beta ? load_f32(g.beta, g.gamma_dtype, k) : 0.0f;
              f[j] = (f[j] - st_a[c]) * st_b[c] * gm + bt;
            } else {
              f[j] = (f[j] / st_b[c]) * gm;
            }
          } else {
            f[j] = 0.0f;
          }
        }
      }
      store8_lds<TC>(&As[buf][r][kc], f);
    }
#pragma unroll
    for (int c = 0; c < CH_B; ++c) {
      const int ci = tid + c * GEMM_THREADS;
      float f[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = to_f32(rb[c].v[j]);
      if (!W_KN) {
        store8_lds<TC>(&Bs[buf][ci / KCH][(ci % KCH) * 8], f);
      } else {
        constexpr int NCH = BN / 8;
        const int kk = ci / NCH, nn = (ci % NCH) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) Bs[buf][nn + j][kk] = from_f32<TC>(f[j]);
      }
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  const int nk = (int)cdiv(K, BK);
  load_tiles(0);
  store_tiles(0, 0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_tiles((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      Frag<TC> af[4], bfr[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = lds_frag<TC>(&As[buf][wm * 64 + t * 16 + fr][ks + fk]);
#pragma unroll
      for (int t = 0; t < 4; ++t) bfr[t] = lds_frag<TC>(&Bs[buf][wn * 64 + t * 16 + fr][ks + fk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) mfma_16x16x32(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < nk) store_tiles(buf ^ 1, (int64_t)(kt + 1) * BK);
    __syncthreads();
  }

  // epilogue
  const int64_t res_rows = g.res_rows > 0 ? g.res_rows : M;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = n0 + wn * 64 + j * 16 + fr;
    if (n >= N) continue;
    const float sc = g.w_scale ? g.w_scale[n] : 1.0f;
    const float bi = g.bias ? load_f32(g.bias, g.bias_dtype, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (m >= M) continue;
        float v = acc[i][j][r] * sc;
        if (g.bias) v += bi;
        if (g.act == ACT_GELU) v = gelu_erf(v);
        if (g.res) v += load_f32(g.res, g.res_dtype, (m % res_rows) * g.ld_res + n);
        store_f32(g.out, g.out_dtype, m * g.ld_out + n, v);
      }
    }
  }
}

}  // namespace cortex

using namespace cortex;

template <class TX, class TC, class TW, bool KN>
static int launch_gemm(const GemmArgs& g, hipStream_t stream) {
  const dim3 grid((unsigned)cdiv(g.N, GEMM_BN), (unsigned)cdiv(g.M, GEMM_BM));
  hipLaunchKernelGGL((gemm_kernel<TX, TC, TW, KN>), grid, dim3(GEMM_THREADS), 0, stream, g);
  CORTEX_CHECK_LAUNCH("gemm_kernel");
  return OK;
}

static int elem_size(int dt) {
  switch (dt) {
    case DT_F32:
    case DT_I32:
      return 4;
    case DT_BF16:
    case DT_F16:
      return 2;
    case DT_I8:
    case DT_U8:
      return 1;
    case DT_I64:
      return 8;
  }
  return 0;
}

// --------------------------------------------------------------------------
// Narrow outputs (N <= 8, e.g. the behaviour head's 512 -> 1 projection): one
// wavefront per row, lanes striding over K, fp32 accumulation.  Operands are
// rounded to bf16 first under bf16 compute, as the MFMA kernels stage them.
// --------------------------------------------------------------------------
constexpr int ROWDOT_MAX_N = 8;

template <class TX, class TW>
__global__ __launch_bounds__(256) void rowdot_kernel(GemmArgs g, int bf16c) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= g.M) return;
  const TX* xr = reinterpret_cast<const TX*>(g.x) + m * g.ld_x;
  const TW* w = reinterpret_cast<const TW*>(g.w);
  float acc[ROWDOT_MAX_N];
#pragma unroll
  for (int n = 0; n < ROWDOT_MAX_N; ++n) acc[n] = 0.0f;
  for (int64_t k = lane; k < g.K; k += 64) {
    float xv = to_f32(xr[k]);
    if (bf16c) xv = (float)(bf16)xv;
#pragma unroll
    for (int n = 0; n < ROWDOT_MAX_N; ++n) {
      if (n < g.N) {
        float wv = to_f32(w[n * g.ld_w + k]);
        if (bf16c) wv = (float)(bf16)wv;
        acc[n] = fmaf(xv, wv, acc[n]);
      }
    }
  }
  const int64_t rr = g.res_rows > 0 ? m % g.res_rows : m;
#pragma unroll
  for (int n = 0; n < ROWDOT_MAX_N; ++n) {
    if (n >= g.N) break;
    float v = wave_sum(acc[n]);
    if (lane != 0) continue;
    if (g.w_scale) v *= g.w_scale[n];
    if (g.bias) v += load_f32(g.bias, g.bias_dtype, n);
    if (g.act == ACT_GELU) v = gelu_erf(v);
    if (g.res) v += load_f32(g.res, g.res_dtype, rr * g.ld_res + n);
    store_f32(g.out, g.out_dtype, m * g.ld_out + n, v);
  }
}

template <class TX, class TW>
static int launch_rowdot(const GemmArgs& g, int bf16c, hipStream_t stream) {
  hipLaunchKernelGGL((rowdot_kernel<TX, TW>), dim3((unsigned)cdiv(g.M, 4)), dim3(256), 0, stream, g, bf16c);
  CORTEX_CHECK_LAUNCH("rowdot_kernel");
  return OK;
}

static int try_rowdot(const GemmArgs& g, int x_dtype, int w_dtype, int w_layout, int compute, hipStream_t stream) {
  if (g.N > ROWDOT_MAX_N || g.norm != NORM_NONE || w_layout != 0 || cdiv(g.M, 4) > 0x7fffffffLL) return 0;
  const int bf16c = compute == DT_BF16 ? 1 : 0;
  if (!bf16c && (x_dtype == DT_BF16 || w_dtype == DT_BF16)) return 0;
  int r = 1;
  if (x_dtype == DT_BF16 && w_dtype == DT_BF16) r = launch_rowdot<bf16, bf16>(g, bf16c, stream);
  else if (x_dtype == DT_BF16 && w_dtype == DT_I8) r = launch_rowdot<bf16, int8_t>(g, bf16c, stream);
  else if (x_dtype == DT_BF16 && w_dtype == DT_F32) r = launch_rowdot<bf16, float>(g, bf16c, stream);
  else if (x_dtype == DT_F32 && w_dtype == DT_BF16) r = launch_rowdot<float, bf16>(g, bf16c, stream);
  else if (x_dtype == DT_F32 && w_dtype == DT_I8) r = launch_rowdot<float, int8_t>(g, bf16c, stream);
  else if (x_dtype == DT_F32 && w_dtype == DT_F32) r = launch_rowdot<float, float>(g, bf16c, stream);
  else return 0;
  return r == OK ? 1 : r;
}

extern "C" {

int cortex_row_stats(int64_t M, int64_t K, int x_dtype, const void* x, int64_t ld_x, int norm, float eps,
                     float* stats, hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0 && K > 0, "cortex_row_stats: need M >= 0 and K > 0");
  CORTEX_CHECK_ARG(norm == NORM_LAYER || norm == NORM_RMS, "cortex_row_stats: norm must be 1 (layer) or 2 (rms)");
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(x && stats && ld_x >= K, "cortex_row_stats: null pointer or ld_x < K");
  const dim3 grid((unsigned)cdiv(M, 4));
  float2* st = reinterpret_cast<float2*>(stats);
  switch (x_dtype) {
    case DT_F32:
      hipLaunchKernelGGL(row_stats_kernel<float>, grid, dim3(256), 0, stream, (const float*)x, M, K, ld_x, norm,
                         eps, st);
      break;
    case DT_BF16:
      hipLaunchKernelGGL(row_stats_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)x, M, K, ld_x, norm,
                         eps, st);
      break;
    default:
      set_error("cortex_row_stats: unsupported x dtype %d", x_dtype);
      return E_UNSUPPORTED;
  }
  CORTEX_CHECK_LAUNCH("row_stats_kernel");
  return OK;
}

int cortex_layer_norm(int64_t M, int64_t K, int x_dtype, const void* x, int64_t ld_x, const void* gamma,
                      const void* beta, int gamma_dtype, float eps, int out_dtype, void* out, int64_t ld_out,
                      hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0 && K > 0, "cortex_layer_norm: need M >= 0 and K > 0");
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(x && out && ld_x >= K && ld_out >= K, "cortex_layer_norm: null pointer or stride < K");
  const dim3 grid((unsigned)cdiv(M, 4));
#define CORTEX_LN(TX, TY)                                                                                   \
  hipLaunchKernelGGL((layer_norm_kernel<TX, TY>), grid, dim3(256), 0, stream, (const TX*)x, M, K, ld_x, gamma, \
                     beta, gamma_dtype, eps, (TY*)out, ld_out)
  if (x_dtype == DT_F32 && out_dtype == DT_F32)
    CORTEX_LN(float, float);
  else if (x_dtype == DT_F32 && out_dtype == DT_BF16)
    CORTEX_LN(float, bf16);
  else if (x_dtype == DT_BF16 && out_dtype == DT_BF16)
    CORTEX_LN(bf16, bf16);
  else if (x_dtype == DT_BF16 && out_dtype == DT_F32)
    CORTEX_LN(bf16, float);
  else {
    set_error("cortex_layer_norm: unsupported dtypes x=%d out=%d", x_dtype, out_dtype);
    return E_UNSUPPORTED;
  }
#undef CORTEX_LN
  CORTEX_CHECK_LAUNCH("layer_norm_kernel");
  return OK;
}

int cortex_norm_linear(int64_t M, int64_t N, int64_t K, int x_dtype, const void* x, int64_t ld_x, int norm,
                       const float* stats, const void* gamma, const void* beta, int gamma_dtype, int compute,
                       int w_dtype, int w_layout, const void* w, int64_t ld_w, const float* w_scale,
                       int bias_dtype, const void* bias, int act, int res_dtype, const void* residual,
                       int64_t ld_res, int64_t res_rows, int out_dtype, void* out, int64_t ld_out,
                       hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "cortex_norm_linear: negative shape");
  if (M == 0 || N == 0) return OK;
  CORTEX_CHECK_ARG(K > 0, "cortex_norm_linear: K must be positive");
  CORTEX_CHECK_ARG(x && w && out, "cortex_norm_linear: null x, w or out");
  CORTEX_CHECK_ARG(ld_x >= K && ld_out >= N, "cortex_norm_linear: ld_x < K or ld_out < N");
  CORTEX_CHECK_ARG(w_layout == 0 ? ld_w >= K : ld_w >= N, "cortex_norm_linear: ld_w too small for the layout");
  CORTEX_CHECK_ARG(norm == NORM_NONE || (stats && gamma), "cortex_norm_linear: norm needs stats and gamma");
  CORTEX_CHECK_ARG(act == ACT_NONE || act == ACT_GELU, "cortex_norm_linear: unknown activation %d", act);
  CORTEX_CHECK_ARG(residual == nullptr || ld_res >= N, "cortex_norm_linear: ld_res < N");
  CORTEX_CHECK_ARG(w_dtype != DT_I8 || w_layout == 0, "cortex_norm_linear: int8 weights must be (N, K)");
  CORTEX_CHECK_ARG(out_dtype == DT_F32 || out_dtype == DT_BF16 || out_dtype == DT_F16,
                   "cortex_norm_linear: unsupported out dtype %d", out_dtype);
  GemmArgs g = {};
  g.M = M;
  g.N = N;
  g.K = K;
  g.x = x;
  g.ld_x = ld_x;
  g.norm = norm;
  g.stats = reinterpret_cast<const float2*>(stats);
  g.gamma = gamma;
  g.beta = beta;
  g.gamma_dtype = gamma_dtype;
  g.w = w;
  g.ld_w = ld_w;
  g.w_scale = w_scale;
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.act = act;
  g.res = residual;
  g.res_dtype = res_dtype;
  g.ld_res = ld_res;
  g.res_rows = res_rows;
  g.out = out;
  g.out_dtype = out_dtype;
  g.ld_out = ld_out;
  CORTEX_CHECK_ARG(cdiv(M, GEMM_BM) <= 65535 && cdiv(N, GEMM_BN) <= 0x7fffffffLL,
                   "cortex_norm_linear: M=%lld exceeds the grid limit", (long long)M);
  if (w_dtype == DT_BF16_FRAG) {  // the weight in MFMA fragment order: the direct-weight residual GEMM alone reads it
    CORTEX_CHECK_ARG(x_dtype == DT_BF16 && compute == DT_BF16 && w_layout == 0 && norm == NORM_NONE &&
                         act == ACT_NONE && residual && res_dtype == DT_F32 && out_dtype == DT_F32 &&
                         (!bias || bias_dtype == DT_F32),
                     "cortex_norm_linear: a fragment-order weight (w_dtype 7) takes bf16 x, an fp32 residual and "
                     "output, no norm and no activation");
    CORTEX_CHECK_ARG(N % 128 == 0 && (K == 1024 || K == 2048 || K == 3072) && M <= 0x7fffffffLL - 128,
                     "cortex_norm_linear: a fragment-order weight needs N a multiple of 128 and K 1024, 2048 or 3072");
    auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    CORTEX_CHECK_ARG(a16(x) && ld_x % 8 == 0 && a16(w) && a16(residual) && ld_res % 4 == 0 && a16(out) &&
                         ld_out % 4 == 0 && (!w_scale || a16(w_scale)) && (!bias || a16(bias)),
                     "cortex_norm_linear: operands must be 16-byte aligned rows");
    return launch_res_dw(g, stream);
  }
  const int xs = elem_size(x_dtype), ws = elem_size(w_dtype);
  const bool vec = ((uintptr_t)x % 16 == 0) && ((ld_x * xs) % 16 == 0) && ((uintptr_t)w % 16 == 0) &&
                   ((ld_w * ws) % 16 == 0) && (ws != 1 || ((uintptr_t)w % 8 == 0 && (ld_w % 8) == 0));
  g.vec = vec ? 1 : 0;
  int fast = try_rowdot(g, x_dtype, w_dtype, w_layout, compute, stream);
  if (fast == 0) fast = try_gemm_bf16(g, x_dtype, w_dtype, w_layout, compute, stream);
  if (fast != 0) return fast > 0 ? OK : fast;
  if (compute == DT_BF16) {
    // fp32 weights are rounded to bf16 (RNE) while staged, i.e. W.to(bfloat16)
    if (x_dtype == DT_BF16) {
      if (w_dtype == DT_I8) return launch_gemm<bf16, bf16, int8_t, false>(g, stream);
      if (w_dtype == DT_BF16)
        return w_layout ? launch_gemm<bf16, bf16, bf16, true>(g, stream) : launch_gemm<bf16, bf16, bf16, false>(g, stream);
      if (w_dtype == DT_F32)
        return w_layout ? launch_gemm<bf16, bf16, float, true>(g, stream)
                        : launch_gemm<bf16, bf16, float, false>(g, stream);
    } else if (x_dtype == DT_F32) {
      if (w_dtype == DT_I8) return launch_gemm<float, bf16, int8_t, false>(g, stream);
      if (w_dtype == DT_BF16)
        return w_layout ? launch_gemm<float, bf16, bf16, true>(g, stream)
                        : launch_gemm<float, bf16, bf16, false>(g, stream);
      if (w_dtype == DT_F32)
        return w_layout ? launch_gemm<float, bf16, float, true>(g, stream)
                        : launch_gemm<float, bf16, float, false>(g, stream);
    }
  } else if (compute == DT_F32) {
    if (x_dtype == DT_F32) {
      if (w_dtype == DT_I8) return launch_gemm<float, float, int8_t, false>(g, stream);
      if (w_dtype == DT_F32)
        return w_layout ? launch_gemm<float, float, float, true>(g, stream)
                        : launch_gemm<float, float, float, false>(g, stream);
    }
  }
  set_error("cortex_norm_linear: unsupported combination x=%d compute=%d w=%d layout=%d", x_dtype, compute, w_dtype,
            w_layout);
  return E_UNSUPPORTED;
}

}  // extern "C"
