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

struct TokLnArgs {
  const float* neuron;
  int64_t n_neuron, ld_neuron;
  const float* time;
  int64_t n_time, ld_time;
  const float* value;
  int64_t n_value, ld_value;
  const int64_t* nid;
  int64_t s_nid;
  const int64_t* tb;
  int64_t s_tb;
  const int64_t* val;
  int64_t s_val;
  int64_t E;
  const int64_t* order;
  const int32_t* ident;  // nullable: *ident != 0 means the plan is the identity (order unused)
  const int64_t* csr_end;
  const float* gamma;
  const float* beta;
  float eps;
  void* out;
  int64_t ld_out;
  int32_t* err;
};

// Row r: lane l holds elements (j/4)*256 + 4l + (j%4), loaded as float4 (coalesced).
template <int EPL>
__global__ __launch_bounds__(256) void ln_rows_kernel(WidenRider wr, const float* __restrict__ x, int64_t M, int64_t ld_x,
                                                       const float* g1, const float* b1, float eps1,
                                                       const float* g2, const float* b2, float eps2, int two,
                                                       bf16* __restrict__ out_bf, int64_t ld_bf,
                                                       float* __restrict__ out_f, int64_t ld_f,
                                                       int8_t* __restrict__ out_q = nullptr, int64_t ld_q = 0,
                                                       float q_inv = 0.0f) {
  constexpr int K = 64 * EPL;
  if ((int)blockIdx.x < wr.blocks) {
    widen_rider_run(wr, (int)blockIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)(blockIdx.x - wr.blocks) * (blockDim.x >> 6) + wave_uniform((int)threadIdx.x >> 6);
  if (m >= M) return;
  const WtOut store_bf(out_bf, M * ld_bf * 2, true), store_f(out_f, M * ld_f * 4, true),
      store_q(out_q, M * ld_q, true);
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
      store_bf(reinterpret_cast<bf16x4*>(out_bf + m * ld_bf + k), b);
    }
    if (out_f) store_f(reinterpret_cast<float4*>(out_f + m * ld_f + k), make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]));
    if (out_q) {  // W8A8: clamp(rint(y * q_inv), -127, 127)
      uint32_t pk = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pk |= (uint32_t)((int)fminf(fmaxf(rintf(v[j + i] * q_inv), -127.0f), 127.0f) & 0xff) << (8 * i);
      store_q(reinterpret_cast<uint32_t*>(out_q + m * ld_q + k), pk);
    }
  }
}


// Normalised rows as the bf16 operand of a linear (the norm half of the fused
// norm + linear, reference cortex/kernels/fused_rmsnorm.py:100-106, and LayerNorm):
//   RMS:   y = (x / sqrt(mean(x^2) + eps)) * gamma
//   layer: y = (x - mean) * (1 / sqrt(var + eps)) * gamma + beta
// in fp32 from bf16 or fp32 x, gamma / beta in fp32 or bf16 (gdt), rounded once to bf16 --
// the same arithmetic as the norm prologue of gemm_kernel.  One wavefront per row,
// lane l holding elements (j / 4) * 256 + 4 l + j % 4.
template <class TX, int EPL>
__global__ __launch_bounds__(256) void norm_rows_kernel(const TX* __restrict__ x, int64_t M, int64_t ld_x, int norm,
                                                        const void* gamma, const void* beta, int gdt, float eps,
                                                        bf16* __restrict__ out, int64_t ld_out) {
  constexpr int K = 64 * EPL;
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (m >= M) return;
  const WtOut store(out, M * ld_out * 2, true);
  const TX* row = x + m * ld_x;
  float v[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    const int k = (j >> 2) * 256 + lane * 4;
    if constexpr (sizeof(TX) == 4) {
      const float4 q = *reinterpret_cast<const float4*>(row + k);
      v[j] = q.x; v[j + 1] = q.y; v[j + 2] = q.z; v[j + 3] = q.w;
    } else {
      const bf16x4 q = *reinterpret_cast<const bf16x4*>(row + k);
      v[j] = (float)q[0]; v[j + 1] = (float)q[1]; v[j + 2] = (float)q[2]; v[j + 3] = (float)q[3];
    }
  }
  float g[EPL], b[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int k = (j >> 2) * 256 + lane * 4 + (j & 3);
    g[j] = !gamma ? 1.0f : gdt == DT_BF16 ? (float)reinterpret_cast<const bf16*>(gamma)[k]
                                          : reinterpret_cast<const float*>(gamma)[k];
    b[j] = !beta ? 0.0f : gdt == DT_BF16 ? (float)reinterpret_cast<const bf16*>(beta)[k]
                                         : reinterpret_cast<const float*>(beta)[k];
  }
  const float inv_k = 1.0f / (float)K;
  if (norm == 2) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) ss += v[j] * v[j];
    const float rms = sqrtf(wave_sum(ss) * inv_k + eps);
#pragma unroll
    for (int j = 0; j < EPL; ++j) v[j] = (v[j] / rms) * g[j];
  } else {
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
    for (int j = 0; j < EPL; ++j) v[j] = (v[j] - mean) * rstd * g[j] + b[j];
  }
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    bf16x4 o;
    o[0] = (bf16)v[j];
    o[1] = (bf16)v[j + 1];
    o[2] = (bf16)v[j + 2];
    o[3] = (bf16)v[j + 3];
    store(reinterpret_cast<bf16x4*>(out + m * ld_out + (j >> 2) * 256 + lane * 4), o);
  }
}

// out[c, r] = in[r, c] for a (R, C) bf16 matrix, through 64 x 64 LDS tiles (the
// (K, N) weight of rms_norm_linear into the (N, K) rows the GEMM streams).  Exact copies.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const bf16* __restrict__ in, int64_t R, int64_t C,
                                                             int64_t ld_in, bf16* __restrict__ out, int64_t ld_out) {
  __shared__ bf16 tile[64][66];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4 threads
#pragma unroll
  for (int i = 0; i < 64; i += 4) {
    const int64_t r = r0 + ty + i, c = c0 + tx;
    if (r < R && c < C) tile[ty + i][tx] = in[r * ld_in + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 64; i += 4) {
    const int64_t c = c0 + ty + i, r = r0 + tx;
    if (r < R && c < C) out[c * ld_out + r] = tile[tx][ty + i];
  }
}

// An (N, K) weight as bf16 in MFMA fragment order, for kernels whose wavefronts each stream
// their own weight rows straight into registers (the direct-weight residual LayerNorm GEMM):
// the 1 KiB block (n16, k32) = n16 * (K / 32) + k32 holds rows 16 n16 .. +15 and K 32 k32 ..
// +31 as 64 lanes x 16 bytes, lane l = row 16 n16 + l % 16, K 32 k32 + 8 (l / 16) .. +7 (the
// operand layout of v_mfma_f32_16x16x32_bf16), so one fragment is one contiguous 1 KiB read.
// Values as cortex_convert writes them (int8 exact, fp32 rounded to nearest even).  One
// thread per 16-byte output chunk.
template <class TW>
__global__ __launch_bounds__(256) void frag_weight_kernel(const TW* __restrict__ w, int64_t ld_w, int64_t K,
                                                          int64_t chunks, bf16* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int64_t b = c >> 6, nkb = K / 32;
  const int l = (int)(c & 63);
  const int64_t n = (b / nkb) * 16 + (l & 15), k = (b % nkb) * 32 + (l >> 4) * 8;
  const TW* src = w + n * ld_w + k;
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = from_f32<bf16>(to_f32(src[j]));
  *reinterpret_cast<bf16x8*>(out + c * 8) = v;
}

// A weight with a norm gain folded into its input columns, as bf16 (N, K) rows:
//   out[n, k] = bf16( float(w[n, k]) * gamma[k] )        (KN = false: (N, K) rows)
//   out[n, k] = bf16( float(w[k, n]) * gamma[k] )        (KN = true: (K, N) rows, through a
//                                                          64 x 64 LDS tile)
// for int8, bf16 or fp32 weights and fp32 or bf16 gamma.  Rows of 64 x 4 threads.
template <class TW, class TG, bool KN>
__global__ __launch_bounds__(256) void fold_gain_kernel(const TW* __restrict__ w, int64_t N, int64_t K, int64_t ld_w,
                                                        const TG* __restrict__ gamma, bf16* __restrict__ out,
                                                        int64_t ld_out) {
  __shared__ float tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  if constexpr (KN) {
#pragma unroll
    for (int i = 0; i < 64; i += 4) {  // rows k of the (K, N) weight, columns n
      const int64_t k = k0 + ty + i, n = n0 + tx;
      if (k < K && n < N) tile[ty + i][tx] = (float)w[k * ld_w + n];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 64; i += 4) {
      const int64_t n = n0 + ty + i, k = k0 + tx;
      if (n < N && k < K) out[n * ld_out + k] = (bf16)(tile[tx][ty + i] * (float)gamma[k]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; i += 4) {
      const int64_t n = n0 + ty + i, k = k0 + tx;
      if (n < N && k < K) out[n * ld_out + k] = (bf16)((float)w[n * ld_w + k] * (float)gamma[k]);
    }
  }
}

// Spike tokens straight to the LayerNorm'd bf16 operand of the cross-attention kv
// projection: row r of the CSR token matrix is
//   x = (neuron_emb[nid[e]] + time_emb[tb[e]]) + value_emb[val[e]]   (fp32, left to right)
// with e = order[r] (rows past *csr_end, or with an index outside its table, are x = 0
// and the latter set bit 1 of err), then LN(x) with gamma/beta/eps is written as bf16.
// The fp32 tokens are never stored.  Same lane layout as ln_rows_kernel.
//
// A row is a chain of dependent loads (order -> indices -> table rows), so each
// wavefront takes TL_ROWS rows and issues every load of one link for all of them
// (and gamma / beta, which depend on nothing) before waiting on any.
constexpr int TL_ROWS = 4;  // 4: 11.1 us at E = 16384, D = 512; 2: 11.4; 1: 11.5

template <int EPL>
__global__ __launch_bounds__(256) void tokenize_ln_kernel(TokLnArgs a, WidenRider wr) {
  constexpr int K = 64 * EPL, R = TL_ROWS;
  if ((int)blockIdx.x < wr.blocks) {
    widen_rider_run(wr, (int)blockIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  // a wavefront's rows, the events they map to and those events' table indices are the same in
  // every lane: kept in scalar registers, as is their address arithmetic
  const int64_t r0 = ((int64_t)(blockIdx.x - wr.blocks) * (blockDim.x >> 6) + wave_uniform((int)threadIdx.x >> 6)) * R;
  if (r0 >= a.E) return;
  const WtOut store(a.out, a.E * a.ld_out * 2, wt_fits(a.E * K * 2));
  const int64_t end = a.csr_end ? *a.csr_end : a.E;
  const bool identity = !a.order || (a.ident && *a.ident);  // sorted events: row r is event r
  int64_t e[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i;
    e[i] = r < a.E ? (identity ? r : wave_uniform(a.order[r])) : -1;
  }
  float4 gm[EPL / 4], bt[EPL / 4];
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    const int k = (j >> 2) * 256 + lane * 4;
    gm[j >> 2] = a.gamma ? *reinterpret_cast<const float4*>(a.gamma + k) : make_float4(1.f, 1.f, 1.f, 1.f);
    bt[j >> 2] = a.beta ? *reinterpret_cast<const float4*>(a.beta + k) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  int64_t i0[R], i1[R], i2[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (r0 + i >= end || e[i] >= a.E) e[i] = -1;  // past the CSR end, or a corrupt order entry
    i0[i] = i1[i] = i2[i] = 0;
    if (e[i] >= 0) {
      i0[i] = wave_uniform(a.nid[e[i] * a.s_nid]);
      i1[i] = wave_uniform(a.tb[e[i] * a.s_tb]);
      i2[i] = wave_uniform(a.val[e[i] * a.s_val]);
    }
  }
  const float* s0[R];
  const float* s1[R];
  const float* s2[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (e[i] >= 0 && (i0[i] < 0 || i0[i] >= a.n_neuron || i1[i] < 0 || i1[i] >= a.n_time || i2[i] < 0 ||
                      i2[i] >= a.n_value)) {
      if (lane == 0 && a.err) atomicOr(a.err, 1);
      e[i] = -1;
    }
    // a row without a valid event reads row 0 of each table and is zeroed below
    s0[i] = a.neuron + (e[i] >= 0 ? i0[i] : 0) * a.ld_neuron;
    s1[i] = a.time + (e[i] >= 0 ? i1[i] : 0) * a.ld_time;
    s2[i] = a.value + (e[i] >= 0 ? i2[i] : 0) * a.ld_value;
  }
  float v[R][EPL];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < EPL; j += 4) {
      const int k = (j >> 2) * 256 + lane * 4;
      const float4 x = *reinterpret_cast<const float4*>(s0[i] + k);
      const float4 y = *reinterpret_cast<const float4*>(s1[i] + k);
      const float4 z = *reinterpret_cast<const float4*>(s2[i] + k);
      v[i][j] = (x.x + y.x) + z.x;
      v[i][j + 1] = (x.y + y.y) + z.y;
      v[i][j + 2] = (x.z + y.z) + z.z;
      v[i][j + 3] = (x.w + y.w) + z.w;
    }
  const float inv_k = 1.0f / (float)K;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (r0 + i >= a.E) break;
    if (e[i] < 0) {
#pragma unroll
      for (int j = 0; j < EPL; ++j) v[i][j] = 0.0f;
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) sum += v[i][j];
    const float mean = wave_sum_dpp(sum) * inv_k;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const float d = v[i][j] - mean;
      ss += d * d;
    }
    const float rstd = 1.0f / sqrtf(wave_sum_dpp(ss) * inv_k + a.eps);
    bf16* out = reinterpret_cast<bf16*>(a.out) + (r0 + i) * a.ld_out;
#pragma unroll
    for (int j = 0; j < EPL; j += 4) {
      const float4 g = gm[j >> 2], b = bt[j >> 2];
      bf16x4 o;
      o[0] = (bf16)((v[i][j] - mean) * rstd * g.x + b.x);
      o[1] = (bf16)((v[i][j + 1] - mean) * rstd * g.y + b.y);
      o[2] = (bf16)((v[i][j + 2] - mean) * rstd * g.z + b.z);
      o[3] = (bf16)((v[i][j + 3] - mean) * rstd * g.w + b.w);
      store(reinterpret_cast<bf16x4*>(out + (j >> 2) * 256 + lane * 4), o);
    }
  }
}

// The whole grid as rider workgroups: the widening on its own launch.
__global__ __launch_bounds__(256) void widen_kernel(WidenRider wr) { widen_rider_run(wr, (int)blockIdx.x); }

// Rider of up to WR_MAX (src int8, dst bf16, count) arrays; arrays with count 0 are dropped.
// frag_k (nullable): per array 0 (dst laid out as src) or the row length K of an (N, K) weight
// whose dst is in MFMA fragment order (a power of two from 64, count a multiple of 16 K).
int make_rider(const char* who, int n, const void* const* src, void* const* dst, const int64_t* count,
               const int64_t* frag_k, WidenRider* r) {
  *r = WidenRider{};
  CORTEX_CHECK_ARG(n >= 0 && n <= WR_MAX, "%s: %d arrays to widen (at most %d)", who, n, WR_MAX);
  if (n == 0) return OK;
  CORTEX_CHECK_ARG(src && dst && count, "%s: null widen list", who);
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    CORTEX_CHECK_ARG(count[i] >= 0 && count[i] % 16 == 0, "%s: widen count %lld is not a multiple of 16", who,
                     (long long)count[i]);
    if (count[i] == 0) continue;
    CORTEX_CHECK_ARG(src[i] && dst[i] && ((uintptr_t)src[i] & 15) == 0 && ((uintptr_t)dst[i] & 15) == 0,
                     "%s: widen arrays must be 16-byte aligned", who);
    const int64_t fk = frag_k ? frag_k[i] : 0;
    CORTEX_CHECK_ARG(fk == 0 || (fk >= 64 && fk <= (1 << 20) && (fk & (fk - 1)) == 0 && count[i] % (16 * fk) == 0),
                     "%s: fragment-order widen needs K a power of two from 64 and count a multiple of 16 K (K %lld)",
                     who, (long long)fk);
    total += count[i];
    r->fk[r->count] = fk ? __builtin_ctzll((unsigned long long)fk) : 0;
    r->src[r->count] = static_cast<const int8_t*>(src[i]);
    r->dst[r->count] = static_cast<bf16*>(dst[i]);
    r->end[r->count] = total;
    ++r->count;
  }
  CORTEX_CHECK_ARG(cdiv(total, WR_CHUNK_SMALL) <= (1 << 24), "%s: %lld elements to widen", who, (long long)total);
  rider_chunk(*r, WR_CHUNK);
  return OK;
}

int widen_launch(const WidenRider& wr, hipStream_t stream) {
  if (wr.blocks == 0) return OK;
  hipLaunchKernelGGL(widen_kernel, dim3((unsigned)wr.blocks), dim3(256), 0, stream, wr);
  CORTEX_CHECK_LAUNCH("widen_kernel");
  return OK;
}

int ln_rows_launch(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma1, const float* beta1,
                   float eps1, const float* gamma2, const float* beta2, float eps2, void* out_bf16, int64_t ld_bf16,
                   float* out_f32, int64_t ld_f32, const WidenRider& wr, hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0, "cortex_ln_rows: negative M");
  if (M == 0 && wr.blocks == 0) return OK;
  CORTEX_CHECK_ARG(M == 0 || (x && (out_bf16 || out_f32)), "cortex_ln_rows: null input or no output");
  CORTEX_CHECK_ARG(K == 256 || K == 512 || K == 768 || K == 1024,
                   "cortex_ln_rows: K=%lld not one of 256, 512, 768, 1024", (long long)K);
  CORTEX_CHECK_ARG(((uintptr_t)x & 15) == 0 && ld_x % 4 == 0, "cortex_ln_rows: x rows must be 16-byte aligned");
  CORTEX_CHECK_ARG(!out_bf16 || (((uintptr_t)out_bf16 & 7) == 0 && ld_bf16 % 4 == 0),
                   "cortex_ln_rows: bf16 output rows must be 8-byte aligned");
  CORTEX_CHECK_ARG(!out_f32 || (((uintptr_t)out_f32 & 15) == 0 && ld_f32 % 4 == 0),
                   "cortex_ln_rows: fp32 output rows must be 16-byte aligned");
  for (const float* p : {gamma1, beta1, gamma2, beta2})
    CORTEX_CHECK_ARG(((uintptr_t)p & 15) == 0, "cortex_ln_rows: gamma/beta must be 16-byte aligned fp32");
  CORTEX_CHECK_ARG(cdiv(M, 4) + wr.blocks <= 0x7fffffffLL, "cortex_ln_rows: M too large");
  const int two = gamma2 != nullptr || beta2 != nullptr;
  const dim3 grid((unsigned)(cdiv(M, 4) + wr.blocks));
#define CORTEX_LNR(EPL)                                                                                              \
  hipLaunchKernelGGL((ln_rows_kernel<EPL>), grid, dim3(256), 0, stream, wr, x, M, ld_x, gamma1, beta1, eps1, gamma2, \
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

int tokenize_ln_launch(int64_t D, const float* neuron_emb, int64_t n_neuron, int64_t ld_neuron, const float* time_emb,
                       int64_t n_time, int64_t ld_time, const float* value_emb, int64_t n_value, int64_t ld_value,
                       const int64_t* neuron_ids, int64_t s_nid, const int64_t* time_bins, int64_t s_tb,
                       const int64_t* values, int64_t s_val, int64_t E, const int64_t* order, const int32_t* identity,
                       const int64_t* csr_end, const float* gamma, const float* beta, float eps, void* out_bf16,
                       int64_t ld_out, int32_t* err_flag, const WidenRider& wr, hipStream_t stream) {
  CORTEX_CHECK_ARG(E >= 0, "cortex_tokenize_ln: negative E");
  if (E == 0 && wr.blocks == 0) return OK;
  CORTEX_CHECK_ARG(D == 256 || D == 512 || D == 768 || D == 1024, "cortex_tokenize_ln: D=%lld not in {256, 512, 768, 1024}",
                   (long long)D);
  CORTEX_CHECK_ARG(E == 0 || (neuron_emb && time_emb && value_emb && neuron_ids && time_bins && values && out_bf16),
                   "cortex_tokenize_ln: null pointer");
  CORTEX_CHECK_ARG(ld_out >= D && ld_neuron >= D && ld_time >= D && ld_value >= D, "cortex_tokenize_ln: ld < D");
  CORTEX_CHECK_ARG(n_neuron > 0 && n_time > 0 && n_value > 0, "cortex_tokenize_ln: empty embedding table");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  CORTEX_CHECK_ARG(al16(neuron_emb) && al16(time_emb) && al16(value_emb) && ld_neuron % 4 == 0 && ld_time % 4 == 0 &&
                       ld_value % 4 == 0 && ((uintptr_t)out_bf16 & 7) == 0 && ld_out % 4 == 0 &&
                       (!gamma || al16(gamma)) && (!beta || al16(beta)),
                   "cortex_tokenize_ln: tables, gamma, beta need 16-byte aligned rows and out 8-byte aligned rows");
  CORTEX_CHECK_ARG(cdiv(E, 4 * TL_ROWS) + wr.blocks <= 0x7fffffffLL, "cortex_tokenize_ln: E too large");
  TokLnArgs a = {neuron_emb, n_neuron, ld_neuron, time_emb, n_time, ld_time, value_emb, n_value, ld_value,
                 neuron_ids, s_nid, time_bins, s_tb, values, s_val, E, order, identity, csr_end, gamma, beta, eps,
                 out_bf16, ld_out, err_flag};
  const dim3 grid((unsigned)(cdiv(E, 4 * TL_ROWS) + wr.blocks));
  switch (D) {
    case 256: hipLaunchKernelGGL(tokenize_ln_kernel<4>, grid, dim3(256), 0, stream, a, wr); break;
    case 512: hipLaunchKernelGGL(tokenize_ln_kernel<8>, grid, dim3(256), 0, stream, a, wr); break;
    case 768: hipLaunchKernelGGL(tokenize_ln_kernel<12>, grid, dim3(256), 0, stream, a, wr); break;
    default: hipLaunchKernelGGL(tokenize_ln_kernel<16>, grid, dim3(256), 0, stream, a, wr); break;
  }
  CORTEX_CHECK_LAUNCH("tokenize_ln_kernel");
  return OK;
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
  return ln_rows_launch(M, K, x, ld_x, gamma1, beta1, eps1, gamma2, beta2, eps2, out_bf16, ld_bf16, out_f32, ld_f32,
                        WidenRider{}, stream);
}

int cortex_ln_rows_widen(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma1, const float* beta1,
                         float eps1, const float* gamma2, const float* beta2, float eps2, void* out_bf16,
                         int64_t ld_bf16, float* out_f32, int64_t ld_f32, int n_widen, const void* const* widen_src,
                         void* const* widen_dst, const int64_t* widen_count, const int64_t* widen_frag_k,
                         hipStream_t stream) {
  WidenRider wr;
  const int st = make_rider("cortex_ln_rows_widen", n_widen, widen_src, widen_dst, widen_count, widen_frag_k, &wr);
  if (st != OK) return st;
  return ln_rows_launch(M, K, x, ld_x, gamma1, beta1, eps1, gamma2, beta2, eps2, out_bf16, ld_bf16, out_f32, ld_f32,
                        wr, stream);
}

int cortex_tokenize_ln(int64_t D, const float* neuron_emb, int64_t n_neuron, int64_t ld_neuron, const float* time_emb,
                       int64_t n_time, int64_t ld_time, const float* value_emb, int64_t n_value, int64_t ld_value,
                       const int64_t* neuron_ids, int64_t s_nid, const int64_t* time_bins, int64_t s_tb,
                       const int64_t* values, int64_t s_val, int64_t E, const int64_t* order, const int32_t* identity,
                       const int64_t* csr_end, const float* gamma, const float* beta, float eps, void* out_bf16,
                       int64_t ld_out, int32_t* err_flag, hipStream_t stream) {
  return tokenize_ln_launch(D, neuron_emb, n_neuron, ld_neuron, time_emb, n_time, ld_time, value_emb, n_value,
                            ld_value, neuron_ids, s_nid, time_bins, s_tb, values, s_val, E, order, identity, csr_end,
                            gamma, beta, eps, out_bf16, ld_out, err_flag, WidenRider{}, stream);
}

int cortex_tokenize_ln_widen(int64_t D, const float* neuron_emb, int64_t n_neuron, int64_t ld_neuron,
                             const float* time_emb, int64_t n_time, int64_t ld_time, const float* value_emb,
                             int64_t n_value, int64_t ld_value, const int64_t* neuron_ids, int64_t s_nid,
                             const int64_t* time_bins, int64_t s_tb, const int64_t* values, int64_t s_val, int64_t E,
                             const int64_t* order, const int32_t* identity, const int64_t* csr_end, const float* gamma,
                             const float* beta, float eps, void* out_bf16, int64_t ld_out, int32_t* err_flag,
                             int n_widen, const void* const* widen_src, void* const* widen_dst,
                             const int64_t* widen_count, const int64_t* widen_frag_k, hipStream_t stream) {
  WidenRider wr;
  const int st =
      make_rider("cortex_tokenize_ln_widen", n_widen, widen_src, widen_dst, widen_count, widen_frag_k, &wr);
  if (st != OK) return st;
  return tokenize_ln_launch(D, neuron_emb, n_neuron, ld_neuron, time_emb, n_time, ld_time, value_emb, n_value,
                            ld_value, neuron_ids, s_nid, time_bins, s_tb, values, s_val, E, order, identity, csr_end,
                            gamma, beta, eps, out_bf16, ld_out, err_flag, wr, stream);
}

int cortex_widen_int8(int n, const void* const* src, void* const* dst, const int64_t* count, const int64_t* frag_k,
                      hipStream_t stream) {
  WidenRider wr;
  const int st = make_rider("cortex_widen_int8", n, src, dst, count, frag_k, &wr);
  if (st != OK) return st;
  return widen_launch(wr, stream);
}

int cortex_norm_rows(int64_t M, int64_t K, int x_dtype, const void* x, int64_t ld_x, int norm, const void* gamma,
                     const void* beta, int gamma_dtype, float eps, void* out, int64_t ld_out, hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0, "cortex_norm_rows: negative M");
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(norm == 1 || norm == 2, "cortex_norm_rows: norm must be 1 (layer) or 2 (rms)");
  CORTEX_CHECK_ARG(K == 256 || K == 512 || K == 768 || K == 1024, "cortex_norm_rows: K=%lld not one of 256, 512, 768, 1024",
                   (long long)K);
  CORTEX_CHECK_ARG(x_dtype == DT_F32 || x_dtype == DT_BF16, "cortex_norm_rows: x must be fp32 or bf16");
  CORTEX_CHECK_ARG(gamma_dtype == DT_F32 || gamma_dtype == DT_BF16, "cortex_norm_rows: gamma must be fp32 or bf16");
  CORTEX_CHECK_ARG(x && out && ld_x >= K && ld_out >= K, "cortex_norm_rows: null pointer or short rows");
  const int xa = x_dtype == DT_F32 ? 15 : 7;
  CORTEX_CHECK_ARG(((uintptr_t)x & xa) == 0 && ld_x % 4 == 0 && ((uintptr_t)out & 7) == 0 && ld_out % 4 == 0,
                   "cortex_norm_rows: x and out rows must be aligned to 4 elements");
  const dim3 grid((unsigned)cdiv(M, 4));
#define CORTEX_NR(TX, EPL)                                                                                      \
  hipLaunchKernelGGL((norm_rows_kernel<TX, EPL>), grid, dim3(256), 0, stream, (const TX*)x, M, ld_x, norm, gamma, \
                     beta, gamma_dtype, eps, (bf16*)out, ld_out)
#define CORTEX_NR_K(TX)              \
  switch (K) {                       \
    case 256: CORTEX_NR(TX, 4); break;  \
    case 512: CORTEX_NR(TX, 8); break;  \
    case 768: CORTEX_NR(TX, 12); break; \
    default: CORTEX_NR(TX, 16); break;  \
  }
  if (x_dtype == DT_F32) {
    CORTEX_NR_K(float)
  } else {
    CORTEX_NR_K(bf16)
  }
#undef CORTEX_NR_K
#undef CORTEX_NR
  CORTEX_CHECK_LAUNCH("norm_rows_kernel");
  return OK;
}

int cortex_transpose_bf16(int64_t R, int64_t C, const void* in, int64_t ld_in, void* out, int64_t ld_out,
                          hipStream_t stream) {
  CORTEX_CHECK_ARG(R >= 0 && C >= 0, "cortex_transpose_bf16: negative size");
  if (R == 0 || C == 0) return OK;
  CORTEX_CHECK_ARG(in && out && ld_in >= C && ld_out >= R, "cortex_transpose_bf16: null pointer or short rows");
  CORTEX_CHECK_ARG(cdiv(R, 64) <= 65535 && cdiv(C, 64) <= 0x7fffffffLL, "cortex_transpose_bf16: too large");
  hipLaunchKernelGGL(transpose_bf16_kernel, dim3((unsigned)cdiv(C, 64), (unsigned)cdiv(R, 64)), dim3(256), 0, stream,
                     (const bf16*)in, R, C, ld_in, (bf16*)out, ld_out);
  CORTEX_CHECK_LAUNCH("transpose_bf16_kernel");
  return OK;
}

int cortex_fold_gain(int64_t N, int64_t K, const void* w, int w_dtype, int kn, int64_t ld_w, const void* gamma,
                     int gamma_dtype, void* out, int64_t ld_out, hipStream_t stream) {
  const char* who = "cortex_fold_gain";
  CORTEX_CHECK_ARG(N >= 0 && K >= 0, "%s: negative size", who);
  if (N == 0 || K == 0) return OK;
  CORTEX_CHECK_ARG(w && gamma && out && ld_out >= K && ld_w >= (kn ? N : K), "%s: null pointer or short rows", who);
  CORTEX_CHECK_ARG(w_dtype == DT_I8 || w_dtype == DT_BF16 || w_dtype == DT_F32, "%s: weight must be int8, bf16 or fp32",
                   who);
  CORTEX_CHECK_ARG(gamma_dtype == DT_F32 || gamma_dtype == DT_BF16, "%s: gamma must be fp32 or bf16", who);
  CORTEX_CHECK_ARG(cdiv(N, 64) <= 65535 && cdiv(K, 64) <= 0x7fffffffLL, "%s: too large", who);
  const dim3 grid((unsigned)cdiv(K, 64), (unsigned)cdiv(N, 64));
#define CORTEX_FOLD(TW, TG, KN)                                                                                    \
  hipLaunchKernelGGL((fold_gain_kernel<TW, TG, KN>), grid, dim3(256), 0, stream, (const TW*)w, N, K, ld_w, \
                     (const TG*)gamma, (bf16*)out, ld_out)
#define CORTEX_FOLD_G(TW)                                                  \
  if (gamma_dtype == DT_F32) {                                             \
    if (kn) CORTEX_FOLD(TW, float, true); else CORTEX_FOLD(TW, float, false); \
  } else {                                                                 \
    if (kn) CORTEX_FOLD(TW, bf16, true); else CORTEX_FOLD(TW, bf16, false);   \
  }
  if (w_dtype == DT_I8) {
    CORTEX_FOLD_G(int8_t)
  } else if (w_dtype == DT_BF16) {
    CORTEX_FOLD_G(bf16)
  } else {
    CORTEX_FOLD_G(float)
  }
#undef CORTEX_FOLD_G
#undef CORTEX_FOLD
  CORTEX_CHECK_LAUNCH("fold_gain_kernel");
  return OK;
}

int cortex_frag_weight(int64_t N, int64_t K, const void* w, int w_dtype, int64_t ld_w, void* out,
                       hipStream_t stream) {
  const char* who = "cortex_frag_weight";
  CORTEX_CHECK_ARG(N >= 0 && K >= 0, "%s: negative size", who);
  if (N == 0 || K == 0) return OK;
  CORTEX_CHECK_ARG(N % 16 == 0 && K % 32 == 0, "%s: N must be a multiple of 16 and K of 32", who);
  CORTEX_CHECK_ARG(w && out && ld_w >= K, "%s: null pointer or short rows", who);
  CORTEX_CHECK_ARG(w_dtype == DT_I8 || w_dtype == DT_BF16 || w_dtype == DT_F32, "%s: weight must be int8, bf16 or fp32",
                   who);
  CORTEX_CHECK_ARG(((uintptr_t)out & 15) == 0, "%s: output must be 16-byte aligned", who);
  const int64_t chunks = N * K / 8;
  CORTEX_CHECK_ARG(cdiv(chunks, (int64_t)256) <= 0x7fffffffLL, "%s: too large", who);
  const dim3 grid((unsigned)cdiv(chunks, (int64_t)256));
  if (w_dtype == DT_I8)
    hipLaunchKernelGGL(frag_weight_kernel<int8_t>, grid, dim3(256), 0, stream, (const int8_t*)w, ld_w, K, chunks,
                       (bf16*)out);
  else if (w_dtype == DT_BF16)
    hipLaunchKernelGGL(frag_weight_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)w, ld_w, K, chunks,
                       (bf16*)out);
  else
    hipLaunchKernelGGL(frag_weight_kernel<float>, grid, dim3(256), 0, stream, (const float*)w, ld_w, K, chunks,
                       (bf16*)out);
  CORTEX_CHECK_LAUNCH("frag_weight_kernel");
  return OK;
}

int cortex_ln_rows_i8(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma, const float* beta,
                      float eps, int8_t* out, int64_t ld_out, float out_scale, hipStream_t stream) {
  CORTEX_CHECK_ARG(M >= 0, "cortex_ln_rows_i8: negative M");
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(x && out && out_scale > 0.0f, "cortex_ln_rows_i8: null pointer or non-positive scale");
  CORTEX_CHECK_ARG(K == 256 || K == 512 || K == 768 || K == 1024,
                   "cortex_ln_rows_i8: K=%lld not one of 256, 512, 768, 1024", (long long)K);
  CORTEX_CHECK_ARG(((uintptr_t)x & 15) == 0 && ld_x % 4 == 0 && ((uintptr_t)out & 3) == 0 && ld_out % 4 == 0 &&
                       ld_out >= K && ld_x >= K,
                   "cortex_ln_rows_i8: rows must be aligned (x 16 bytes, out 4 bytes)");
  for (const float* p : {gamma, beta})
    CORTEX_CHECK_ARG(((uintptr_t)p & 15) == 0, "cortex_ln_rows_i8: gamma/beta must be 16-byte aligned fp32");
  const dim3 grid((unsigned)cdiv(M, 4));
  const float inv = 1.0f / out_scale;
#define CORTEX_LNQ(EPL)                                                                                              \
  hipLaunchKernelGGL((ln_rows_kernel<EPL>), grid, dim3(256), 0, stream, WidenRider{}, x, M, ld_x, gamma, beta, eps, \
                     nullptr, nullptr, 0.0f, 0, nullptr, 0, nullptr, 0, out, ld_out, inv)
  switch (K) {
    case 256: CORTEX_LNQ(4); break;
    case 512: CORTEX_LNQ(8); break;
    case 768: CORTEX_LNQ(12); break;
    default: CORTEX_LNQ(16); break;
  }
#undef CORTEX_LNQ
  CORTEX_CHECK_LAUNCH("ln_rows_kernel (int8)");
  return OK;
}

}  // extern "C"
