// Behaviour head of the Cortex forward (reference cortex/models/cortex.py:29-53), fused.
//
// The head is  out[b, q] = w_out . concat_h( softmax_l(q_h . k_{l,h} / sqrt(Dh)) V_h )
// with k, v = W_kv n_l and n_l = LN_head(LN_final(x_{b,l})) (the encoder's final norm
// and the head's own norm).  Every factor but n is batch-invariant, so the weights are
// folded into the queries and the output projection once per parameter state:
//
//   a_{q,h} = W_k[h]^T q_h * log2(e) / sqrt(Dh)   scores in the exp2 domain: s = a . n_l
//   c_h     = W_v[h]^T w_out[h]                    t_{l,h} = c_h . n_l
//   out[b,q] = sum_h  sum_l 2^(s_{q,h,l}) t_{l,h}  /  sum_l 2^(s_{q,h,l})
//
// (softmax weights sum to one, so the V projection and w_out commute with the sum over
// latents).  The head then reads each latent row once: two LayerNorms in registers,
// then one 16x16x32 MFMA pair per 16 latents against the 32 folded rows
// [a_{q,h} (Q*H rows) | c_{h(r)} for each of those rows], then an online softmax
// that stays in the lane holding both s and t of a (row, latent) pair.  Latents are
// split over workgroups (16 per workgroup, 4 rows per wavefront, so every CU gets work
// at B = 32); a second small launch merges the split partials per sample.  The kv projection
// (B*L x 2D x D), the attention and the output projection disappear.
#include <hip/hip_runtime.h>

#include "common.h"

namespace cortex {

namespace {

constexpr int HD_WAVES = 4;
constexpr int HD_ROWS = 32;  // folded rows: 16 query-head rows + their 16 value rows

struct PrepArgs {
  const bf16* qv;  // (Q, D) projected behaviour queries
  int64_t ld_q;
  int Q, H, Dh, D;
  const bf16* wkv;  // (2D, D) kv weight (bf16 image), rows [0, D) keys, [D, 2D) values
  const float* s_kv;  // (2D) per-row scale or null
  int64_t ld_w;
  const bf16* wout;  // (1, D) output weight (bf16 image)
  const float* s_out;  // (1) scale or null
  float qscale;
  bf16* ac;  // (32, D)
};

__global__ __launch_bounds__(256) void head_prep_kernel(PrepArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)HD_ROWS * a.D) return;
  const int r = (int)(idx / a.D), j = (int)(idx % a.D);
  const int QH = a.Q * a.H;
  float acc = 0.0f;
  if (r < QH) {
    const int q = r / a.H, h = r % a.H;
    for (int d = 0; d < a.Dh; ++d) {
      const int row = h * a.Dh + d;
      const float sc = a.s_kv ? a.s_kv[row] : 1.0f;
      acc += (float)a.qv[q * a.ld_q + row] * sc * (float)a.wkv[(int64_t)row * a.ld_w + j];
    }
    acc *= a.qscale;
  } else if (r >= 16 && r - 16 < QH) {
    const int h = (r - 16) % a.H;
    const float so = a.s_out ? a.s_out[0] : 1.0f;
    for (int d = 0; d < a.Dh; ++d) {
      const int row = a.D + h * a.Dh + d;
      const float sc = a.s_kv ? a.s_kv[row] : 1.0f;
      acc += (float)a.wout[h * a.Dh + d] * so * sc * (float)a.wkv[(int64_t)row * a.ld_w + j];
    }
  }
  a.ac[idx] = (bf16)acc;
}

struct HeadArgs {
  const float* x;  // (B*L, D) fp32 latents, row b*L + l
  int64_t ld_x;
  int64_t L;
  int Q, H;
  const float *g1, *b1, *g2, *b2;
  float eps1, eps2;
  const bf16* ac;  // (32, D)
  float* part;     // (B, n_split, 16, 3) online-softmax partials (max, sum, weighted sum)
  int n_split;
  float* out;      // (B, Q)
};

// The head runs one wavefront per SIMD, with nothing else to hide reduction latency behind:
// its row sums use the DPP reduction (wave_sum_dpp), not LDS shuffles.
__device__ __forceinline__ float hd_wave_sum(float v) { return wave_sum_dpp(v); }

// LayerNorm parameters of one lane's EPL columns (k = (j / 4) * 256 + lane * 4 + j % 4)
template <int EPL>
struct LnRegs {
  float g[EPL], b[EPL];
  __device__ void load(const float* gamma, const float* beta, int lane) {
#pragma unroll
    for (int j = 0; j < EPL; j += 4) {
      const int k = (j >> 2) * 256 + lane * 4;
      const float4 gm = *reinterpret_cast<const float4*>(gamma + k);
      const float4 be = *reinterpret_cast<const float4*>(beta + k);
      g[j] = gm.x, g[j + 1] = gm.y, g[j + 2] = gm.z, g[j + 3] = gm.w;
      b[j] = be.x, b[j + 1] = be.y, b[j + 2] = be.z, b[j + 3] = be.w;
    }
  }
};

// LayerNorm of a row spread over the wave (EPL values per lane); the rounding of the
// result to bf16 follows, so the hardware reciprocal square root is accurate enough.
template <int EPL>
__device__ __forceinline__ void hd_ln(float (&v)[EPL], float inv_k, float eps, const LnRegs<EPL>& p) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) s += v[j];
  const float mean = hd_wave_sum(s) * inv_k;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    v[j] -= mean;
    ss += v[j] * v[j];
  }
  const float rstd = __builtin_amdgcn_rsqf(hd_wave_sum(ss) * inv_k + eps);
#pragma unroll
  for (int j = 0; j < EPL; ++j) v[j] = v[j] * rstd * p.g[j] + p.b[j];
}

// (m, s, t) of one online-softmax stream: running max, sum of 2^(x - m), sum of 2^(x - m) t
__device__ __forceinline__ void hd_merge(float& m, float& s, float& t, float m2, float s2, float t2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  const float f1 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
  const float f2 = m2 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m2 - mn);
  s = s * f1 + s2 * f2;
  t = t * f1 + t2 * f2;
  m = mn;
}

// Grid (B, n_split): workgroup (b, y) takes the 16 latents [16 y, 16 y + 16) of sample
// b.  Each wavefront normalises 4 of the rows into the shared stage; wavefront 0 then
// multiplies the tile against the folded rows (fragments read straight from global
// memory, where they are L2-resident) and writes the tile's online-softmax partials.
// D = 64 EPL.
template <int EPL>
__global__ __launch_bounds__(64 * HD_WAVES) void head_partial_kernel(HeadArgs a) {
  constexpr int D = 64 * EPL;
  constexpr int PITCH = D + 8;  // bf16 elements per LDS row: 16-byte skew per row
  constexpr int RPW = 16 / HD_WAVES;  // rows per wavefront
  __shared__ __attribute__((aligned(16))) bf16 stage[16 * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.x;
  const int64_t l0 = (int64_t)blockIdx.y * 16;
  // wavefront 0's folded-row fragments, in flight while the rows are normalised
  bf16x8 af[2][D / 32];
  if (w == 0) {
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      af[0][ks] = *reinterpret_cast<const bf16x8*>(a.ac + fr * D + ks * 32 + g * 8);
      af[1][ks] = *reinterpret_cast<const bf16x8*>(a.ac + (16 + fr) * D + ks * 32 + g * 8);
    }
  }

  {
    float v[RPW][EPL];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const int64_t l = min(l0 + w * RPW + rr, a.L - 1);  // rows past L: a valid row, never used
      const float* xr = a.x + (b * a.L + l) * a.ld_x;
#pragma unroll
      for (int j = 0; j < EPL; j += 4) {
        const float4 q = *reinterpret_cast<const float4*>(xr + (j >> 2) * 256 + lane * 4);
        v[rr][j] = q.x, v[rr][j + 1] = q.y, v[rr][j + 2] = q.z, v[rr][j + 3] = q.w;
      }
    }
    LnRegs<EPL> p1, p2;
    p1.load(a.g1, a.b1, lane);
    p2.load(a.g2, a.b2, lane);
    const float inv_k = 1.0f / (float)D;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      hd_ln<EPL>(v[rr], inv_k, a.eps1, p1);
      hd_ln<EPL>(v[rr], inv_k, a.eps2, p2);
#pragma unroll
      for (int j = 0; j < EPL; j += 4) {
        bf16x4 o;
        o[0] = (bf16)v[rr][j];
        o[1] = (bf16)v[rr][j + 1];
        o[2] = (bf16)v[rr][j + 2];
        o[3] = (bf16)v[rr][j + 3];
        *reinterpret_cast<bf16x4*>(stage + (w * RPW + rr) * PITCH + (j >> 2) * 256 + lane * 4) = o;
      }
    }
  }
  __syncthreads();
  if (w != 0) return;
  f32x4 acc0 = (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    const bf16x8 nf = *reinterpret_cast<const bf16x8*>(stage + fr * PITCH + ks * 32 + g * 8);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[0][ks], nf, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[1][ks], nf, acc1, 0, 0, 0);
  }
  // acc0[i] = s of folded row 4g+i at latent l0+fr, acc1[i] = its t; combine the 16
  // latents of each lane group
  float m_run[4], s_run[4], t_run[4];
  const bool valid = l0 + fr < a.L;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = valid ? acc0[i] : -INFINITY;
    s_run[i] = valid ? 1.0f : 0.0f;
    t_run[i] = valid ? acc1[i] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // DPP exchange inside each 16-lane row (as hd_wave_sum)
    hd_merge(m_run[i], s_run[i], t_run[i], dpp_mov<0xB1>(m_run[i]), dpp_mov<0xB1>(s_run[i]), dpp_mov<0xB1>(t_run[i]));
    hd_merge(m_run[i], s_run[i], t_run[i], dpp_mov<0x4E>(m_run[i]), dpp_mov<0x4E>(s_run[i]), dpp_mov<0x4E>(t_run[i]));
    hd_merge(m_run[i], s_run[i], t_run[i], dpp_mov<0x124>(m_run[i]), dpp_mov<0x124>(s_run[i]),
             dpp_mov<0x124>(t_run[i]));
    hd_merge(m_run[i], s_run[i], t_run[i], dpp_mov<0x128>(m_run[i]), dpp_mov<0x128>(s_run[i]),
             dpp_mov<0x128>(t_run[i]));
  }
  if (fr == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* p = a.part + ((b * a.n_split + blockIdx.y) * 16 + 4 * g + i) * 3;
      p[0] = m_run[i];
      p[1] = s_run[i];
      p[2] = t_run[i];
    }
  }
}

// One workgroup per sample: thread (row r, group y0) merges splits y0, y0 + 16, ... with
// every load issued up front, the 16 groups are merged through LDS, then the heads summed.
__global__ __launch_bounds__(256) void head_merge_kernel(HeadArgs a) {
  __shared__ float grp[16][16][3];
  __shared__ float res[16];
  const int64_t b = blockIdx.x;
  const int r = threadIdx.x & 15, y0 = threadIdx.x >> 4;
  float m = -INFINITY, s = 0.0f, t = 0.0f;
  for (int y = y0; y < a.n_split; y += 16) {
    const float* p = a.part + ((b * a.n_split + y) * 16 + r) * 3;
    hd_merge(m, s, t, p[0], p[1], p[2]);
  }
  grp[y0][r][0] = m;
  grp[y0][r][1] = s;
  grp[y0][r][2] = t;
  __syncthreads();
  const int QH = a.Q * a.H;
  if (threadIdx.x < QH) {
    float mm = grp[0][r][0], ss = grp[0][r][1], tt = grp[0][r][2];
    for (int yy = 1; yy < 16; ++yy) hd_merge(mm, ss, tt, grp[yy][r][0], grp[yy][r][1], grp[yy][r][2]);
    res[r] = ss > 0.0f ? tt / ss : 0.0f;
  }
  __syncthreads();
  if (threadIdx.x < a.Q) {
    float o = 0.0f;
    for (int h = 0; h < a.H; ++h) o += res[threadIdx.x * a.H + h];
    a.out[b * a.Q + threadIdx.x] = o;
  }
}

// Masked-spike head (reference cortex/models/cortex.py:56-69): the mean over a sample's
// L latent rows (after an optional LayerNorm, the encoder's final norm) and a small
// linear N x D (+ bias) on that mean.  One workgroup per sample; wavefront w takes rows
// w, w + 4, ... and keeps its column sums in registers (EPL = D / 64 per lane, the
// ln_regs layout), so rows are read once and no barrier sits inside the row loop.
struct PoolArgs {
  const float* x;
  int64_t ld_x, L;
  const float* gamma;  // LayerNorm applied to each row first when non-null
  const float* beta;
  float eps;
  int N;
  int w_dtype;       // DT_F32 or DT_I8
  const void* w;     // (N, D) rows, ld_w apart; null: pooled rows only
  int64_t ld_w;
  const float* w_scale;  // (N) per-row scale of an int8 weight
  const float* bias;     // (N) or null
  float* pooled;         // (B, D) mean rows, or null
  float* out;            // (B, N)
};

template <int EPL>
__global__ __launch_bounds__(256) void pooled_linear_kernel(PoolArgs a) {
  constexpr int D = EPL * 64;
  __shared__ float part[4][D];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t b = blockIdx.x;
  float acc[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) acc[j] = 0.0f;
  const float inv_k = 1.0f / (float)D;
  for (int64_t l = w; l < a.L; l += 4) {
    const float* row = a.x + (b * a.L + l) * a.ld_x;
    float v[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j += 4) {
      const float4 t = *reinterpret_cast<const float4*>(row + (j >> 2) * 256 + lane * 4);
      v[j] = t.x;
      v[j + 1] = t.y;
      v[j + 2] = t.z;
      v[j + 3] = t.w;
    }
    if (a.gamma) ln_regs<EPL>(v, inv_k, a.eps, a.gamma, a.beta, lane);
#pragma unroll
    for (int j = 0; j < EPL; ++j) acc[j] += v[j];
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) part[w][(j >> 2) * 256 + lane * 4 + (j & 3)] = acc[j];
  __syncthreads();
  const float inv_l = 1.0f / (float)a.L;
  for (int k = threadIdx.x; k < D; k += 256) {
    const float m = ((part[0][k] + part[1][k]) + (part[2][k] + part[3][k])) * inv_l;
    part[0][k] = m;
    if (a.pooled) a.pooled[b * D + k] = m;
  }
  __syncthreads();
  if (!a.w) return;
  for (int n = w; n < a.N; n += 4) {
    float dot = 0.0f;
    if (a.w_dtype == DT_I8) {
      const int8_t* wr = reinterpret_cast<const int8_t*>(a.w) + (int64_t)n * a.ld_w;
      const float sc = a.w_scale[n];
      for (int k = lane; k < D; k += 64) dot = fmaf(part[0][k], (float)(int)wr[k] * sc, dot);
    } else {
      const float* wr = reinterpret_cast<const float*>(a.w) + (int64_t)n * a.ld_w;
      for (int k = lane; k < D; k += 64) dot = fmaf(part[0][k], wr[k], dot);
    }
    dot = wave_sum(dot);
    if (lane == 0) a.out[b * a.N + n] = dot + (a.bias ? a.bias[n] : 0.0f);
  }
}

bool al(const void* p, int n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

}  // namespace cortex

using namespace cortex;

extern "C" int cortex_head_prep(const void* qv, int64_t ld_q, int64_t Q, int64_t H, int64_t D, const void* wkv,
                                const float* s_kv, int64_t ld_w, const void* wout, const float* s_out, void* ac,
                                hipStream_t stream) {
  CORTEX_CHECK_ARG(Q >= 1 && H >= 1 && Q * H <= 16 && D > 0 && D % H == 0,
                   "cortex_head_prep: need 1 <= Q*H <= 16 and H dividing D");
  CORTEX_CHECK_ARG(qv && wkv && wout && ac, "cortex_head_prep: null pointer");
  CORTEX_CHECK_ARG(ld_q >= D && ld_w >= D, "cortex_head_prep: row strides must be >= D");
  const int Dh = (int)(D / H);
  PrepArgs a{reinterpret_cast<const bf16*>(qv), ld_q, (int)Q, (int)H, Dh, (int)D,
             reinterpret_cast<const bf16*>(wkv), s_kv, ld_w, reinterpret_cast<const bf16*>(wout), s_out,
             1.4426950408889634f / sqrtf((float)Dh), reinterpret_cast<bf16*>(ac)};
  const int64_t n = HD_ROWS * D;
  hipLaunchKernelGGL(head_prep_kernel, dim3((unsigned)cdiv(n, (int64_t)256)), dim3(256), 0, stream, a);
  CORTEX_CHECK_LAUNCH("head_prep_kernel");
  return OK;
}

extern "C" int64_t cortex_behavior_head_workspace_bytes(int64_t B, int64_t L) {
  if (B <= 0 || L <= 0) return 0;
  return B * cdiv(L, (int64_t)16) * 16 * 3 * (int64_t)sizeof(float);
}

extern "C" int cortex_behavior_head(const float* x, int64_t ld_x, int64_t B, int64_t L, int64_t D, int64_t Q,
                                    int64_t H, const float* gamma1, const float* beta1, float eps1,
                                    const float* gamma2, const float* beta2, float eps2, const void* ac, float* out,
                                    void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  CORTEX_CHECK_ARG(B >= 0 && L >= 1 && Q >= 1 && H >= 1 && Q * H <= 16, "cortex_behavior_head: bad sizes");
  CORTEX_CHECK_ARG(D == 256 || D == 512 || D == 768, "cortex_behavior_head: D must be 256, 512 or 768");
  if (B == 0) return OK;
  CORTEX_CHECK_ARG(x && gamma1 && beta1 && gamma2 && beta2 && ac && out, "cortex_behavior_head: null pointer");
  CORTEX_CHECK_ARG(ld_x >= D && ld_x % 4 == 0 && al(x, 16) && al(ac, 16) && al(gamma1, 16) && al(beta1, 16) &&
                       al(gamma2, 16) && al(beta2, 16),
                   "cortex_behavior_head: rows and parameters must be 16-byte aligned");
  const int64_t need = cortex_behavior_head_workspace_bytes(B, L);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("cortex_behavior_head: workspace of %lld bytes is smaller than the required %lld",
              (long long)workspace_bytes, (long long)need);
    return E_WORKSPACE;
  }
  const int64_t n_split = cdiv(L, (int64_t)16);
  CORTEX_CHECK_ARG(B <= 0x7fffffffLL && n_split <= 65535, "cortex_behavior_head: B or L too large");
  HeadArgs a{x, ld_x, L, (int)Q, (int)H, gamma1, beta1, gamma2, beta2, eps1, eps2,
             reinterpret_cast<const bf16*>(ac), reinterpret_cast<float*>(workspace), (int)n_split, out};
  const dim3 grid((unsigned)B, (unsigned)n_split), block(64 * HD_WAVES);
  switch (D) {
    case 256: hipLaunchKernelGGL(head_partial_kernel<4>, grid, block, 0, stream, a); break;
    case 512: hipLaunchKernelGGL(head_partial_kernel<8>, grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL(head_partial_kernel<12>, grid, block, 0, stream, a); break;
  }
  CORTEX_CHECK_LAUNCH("head_partial_kernel");
  hipLaunchKernelGGL(head_merge_kernel, dim3((unsigned)B), dim3(256), 0, stream, a);
  CORTEX_CHECK_LAUNCH("head_merge_kernel");
  return OK;
}

extern "C" int cortex_pooled_linear(const float* x, int64_t ld_x, int64_t B, int64_t L, int64_t D, const float* gamma,
                                    const float* beta, float eps, int64_t N, int w_dtype, const void* w,
                                    int64_t ld_w, const float* w_scale, const float* bias, float* pooled,
                                    float* out, hipStream_t stream) {
  CORTEX_CHECK_ARG(B >= 0 && L >= 1 && N >= 0, "cortex_pooled_linear: bad sizes");
  CORTEX_CHECK_ARG(D == 256 || D == 512 || D == 768 || D == 1024, "cortex_pooled_linear: D must be 256, 512, 768 or 1024");
  if (B == 0) return OK;
  CORTEX_CHECK_ARG(x && ld_x >= D && ld_x % 4 == 0 && al(x, 16), "cortex_pooled_linear: x must be 16-byte aligned rows");
  CORTEX_CHECK_ARG(!gamma || (beta && al(gamma, 16) && al(beta, 16)),
                   "cortex_pooled_linear: LayerNorm needs 16-byte aligned gamma and beta");
  CORTEX_CHECK_ARG(w || pooled, "cortex_pooled_linear: nothing to write (no weight and no pooled output)");
  if (w) {
    CORTEX_CHECK_ARG(out && ld_w >= D, "cortex_pooled_linear: null out or weight stride below D");
    CORTEX_CHECK_ARG(w_dtype == DT_F32 || (w_dtype == DT_I8 && w_scale),
                     "cortex_pooled_linear: weight must be fp32, or int8 with a per-row scale");
  }
  CORTEX_CHECK_ARG(B <= 0x7fffffffLL && N <= 0x7fffffffLL, "cortex_pooled_linear: B or N too large");
  PoolArgs a{x, ld_x, L, gamma, beta, eps, (int)N, w_dtype, w, ld_w, w_scale, bias, pooled, out};
  const dim3 grid((unsigned)B), block(256);
  switch (D) {
    case 256: hipLaunchKernelGGL(pooled_linear_kernel<4>, grid, block, 0, stream, a); break;
    case 512: hipLaunchKernelGGL(pooled_linear_kernel<8>, grid, block, 0, stream, a); break;
    case 768: hipLaunchKernelGGL(pooled_linear_kernel<12>, grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL(pooled_linear_kernel<16>, grid, block, 0, stream, a); break;
  }
  CORTEX_CHECK_LAUNCH("pooled_linear_kernel");
  return OK;
}
