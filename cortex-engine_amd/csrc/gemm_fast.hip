// Fast-path fused norm + GEMM for the Cortex forward on gfx950 (bf16 MFMA).
//
// Same contract as the general kernel in norm_gemm.hip, specialised at compile time
// for the shapes the model runs (K a multiple of BK, 16-byte aligned rows):
//   A  bf16 rows, or fp32 rows normalised while staged (LayerNorm or RMSNorm with
//      precomputed per-row statistics, fp32 gamma/beta) and rounded to bf16;
//   W  int8 (N, K) widened exactly to bf16 while staged, or fp32 (N, K) rounded;
//   epilogue  acc * scale[n] (+bias) (-> GELU) (+ fp32 residual), bf16/fp32 out.
//
// Tiling is a template: a BM x BN workgroup tile split over WM x WN wavefronts,
// each wavefront owning (BM/WM) x (BN/WN) as 16x16 v_mfma_f32_16x16x32_bf16 tiles;
// K steps of BK through two LDS stages with register prefetch of the next step.
// The epilogue stages the finished tile through LDS so that residual reads and
// output writes are full 16-byte rows (coalesced), not 16-lane column strips.
// Workgroups are renumbered so that each XCD (8 per MI355X, round-robin dispatch)
// owns a contiguous band of output rows and keeps that band of A in its own L2.
#include <hip/hip_runtime.h>

#include "common.h"
#include "gemm.h"

namespace cortex {

namespace {

template <class T>
struct RawA;
template <>
struct RawA<bf16> {
  uint4 v;
};
template <>
struct RawA<float> {
  uint4 v[2];
};
template <class T>
struct RawW;
template <>
struct RawW<int8_t> {
  uint2 v;
};
template <>
struct RawW<float> {
  uint4 v[2];
};

__device__ __forceinline__ void unpack(const RawA<bf16>& r, float (&f)[8]) {
  const bf16* p = reinterpret_cast<const bf16*>(&r.v);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = (float)p[j];
}
__device__ __forceinline__ void unpack(const RawA<float>& r, float (&f)[8]) {
  const float* p = reinterpret_cast<const float*>(r.v);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = p[j];
}
__device__ __forceinline__ void unpack(const RawW<int8_t>& r, float (&f)[8]) {
  const int8_t* p = reinterpret_cast<const int8_t*>(&r.v);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = (float)(int)p[j];
}
__device__ __forceinline__ void unpack(const RawW<float>& r, float (&f)[8]) {
  const float* p = reinterpret_cast<const float*>(r.v);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = p[j];
}

// Unconditional 16/8-byte loads: out-of-range rows are clamped to a valid row by the
// caller (their products only reach output rows/columns the epilogue never stores),
// so the prefetch has no exec-masked branches for the compiler to serialise on.
__device__ __forceinline__ void gload(RawA<bf16>& r, const bf16* p) { r.v = *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void gload(RawA<float>& r, const float* p) {
  r.v[0] = reinterpret_cast<const uint4*>(p)[0];
  r.v[1] = reinterpret_cast<const uint4*>(p)[1];
}
__device__ __forceinline__ void gload(RawW<int8_t>& r, const int8_t* p) { r.v = *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ void gload(RawW<float>& r, const float* p) {
  r.v[0] = reinterpret_cast<const uint4*>(p)[0];
  r.v[1] = reinterpret_cast<const uint4*>(p)[1];
}

__device__ __forceinline__ void st_bf16x8(bf16* dst, const float (&f)[8]) {
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (bf16)f[j];
  *reinterpret_cast<bf16x8*>(dst) = v;
}

// the same 8 values as an output row chunk (global memory only; written through as `store` says)
__device__ __forceinline__ void st_bf16x8_out(bf16* dst, const float (&f)[8], const WtOut& store) {
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (bf16)f[j];
  store(reinterpret_cast<bf16x8*>(dst), v);
}

template <int BM_, int BN_, int WM_, int WN_, int BK_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int LDK = BK + 8;                    // bf16 row pitch of the operand stages
  static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  static constexpr int KCH = BK / 8;                    // 8-element chunks per tile row
  static constexpr int CA = BM * KCH / THREADS, CB = BN * KCH / THREADS;
  static constexpr int RSTRIDE = THREADS / KCH;         // rows between a thread's chunks
  static constexpr int OPER_BYTES = 2 * (BM + BN) * LDK * 2;
  static constexpr int EPI_LD = BN + 4;                 // fp32 row pitch of the epilogue stage
  static constexpr int EPI_BYTES = WM * 16 * EPI_LD * 4;
  static constexpr int LDS_BYTES = OPER_BYTES > EPI_BYTES ? OPER_BYTES : EPI_BYTES;
  static_assert(CA >= 1 && CB >= 1 && BM * KCH % THREADS == 0 && BN * KCH % THREADS == 0, "staging split");
  static_assert(TM >= 1 && TN >= 1, "wave tile");
};

template <class TL, class TX, class TW, int NORM, int ACT, bool RES, class TOUT>
__global__ __launch_bounds__(TL::THREADS, 2) void gemm_fast_kernel(GemmArgs g) {
  constexpr int BM = TL::BM, BN = TL::BN, BK = TL::BK, LDK = TL::LDK, TM = TL::TM, TN = TL::TN;
  constexpr int CA = TL::CA, CB = TL::CB, RS = TL::RSTRIDE;
  __shared__ __attribute__((aligned(16))) unsigned char smem[TL::LDS_BYTES];
  bf16(*As)[BM][LDK] = reinterpret_cast<bf16(*)[BM][LDK]>(smem);
  bf16(*Bs)[BN][LDK] = reinterpret_cast<bf16(*)[BN][LDK]>(smem + 2 * BM * LDK * 2);

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / TL::WN, wn = wid % TL::WN;
  const int nbx = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + nbx * blockIdx.y, total);
  const int m0 = (id / nbx) * BM, n0 = (id % nbx) * BN;
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const TX* __restrict__ X = reinterpret_cast<const TX*>(g.x);
  const TW* __restrict__ W = reinterpret_cast<const TW*>(g.w);

  const int srow = tid / TL::KCH, skc = (tid % TL::KCH) * 8;
  float s_a[CA], s_b[CA];
#pragma unroll
  for (int c = 0; c < CA; ++c) {
    s_a[c] = 0.0f;
    s_b[c] = 1.0f;
    const int m = m0 + srow + RS * c;
    if (NORM != NORM_NONE && m < M) {
      const float2 st = g.stats[m];
      s_a[c] = st.x;
      s_b[c] = NORM == NORM_RMS ? 1.0f / st.y : st.y;
    }
  }

  // two register sets: tile k+2 is loaded while tile k is multiplied and tile k+1
  // (loaded one step earlier) is written to LDS, so each load has two MFMA phases
  // to arrive
  struct RegSet {
    RawA<TX> a[CA];
    RawW<TW> b[CB];
    float4 gm[2], bt[2];
  };
  RegSet rs0, rs1;
  const float* gamma = reinterpret_cast<const float*>(g.gamma);
  const float* beta = reinterpret_cast<const float*>(g.beta);

  // per-thread row bases (rows past M / N clamped to the last valid row)
  const TX* xrow[CA];
  const TW* wrow_p[CB];
#pragma unroll
  for (int c = 0; c < CA; ++c) xrow[c] = X + (int64_t)min(m0 + srow + RS * c, M - 1) * g.ld_x + skc;
#pragma unroll
  for (int c = 0; c < CB; ++c) wrow_p[c] = W + (int64_t)min(n0 + srow + RS * c, N - 1) * g.ld_w + skc;

  auto load_tiles = [&](RegSet& rs, int k0) {
#pragma unroll
    for (int c = 0; c < CA; ++c) gload(rs.a[c], xrow[c] + k0);
#pragma unroll
    for (int c = 0; c < CB; ++c) gload(rs.b[c], wrow_p[c] + k0);
    if (NORM != NORM_NONE) {
      rs.gm[0] = *reinterpret_cast<const float4*>(gamma + k0 + skc);
      rs.gm[1] = *reinterpret_cast<const float4*>(gamma + k0 + skc + 4);
      if (NORM == NORM_LAYER && beta) {
        rs.bt[0] = *reinterpret_cast<const float4*>(beta + k0 + skc);
        rs.bt[1] = *reinterpret_cast<const float4*>(beta + k0 + skc + 4);
      } else {
        rs.bt[0] = rs.bt[1] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };

  auto store_tiles = [&](const RegSet& rs, int buf) {
#pragma unroll
    for (int c = 0; c < CA; ++c) {
      bf16* dst = &As[buf][srow + RS * c][skc];
      if constexpr (sizeof(TX) == 2 && NORM == NORM_NONE) {
        *reinterpret_cast<uint4*>(dst) = rs.a[c].v;  // bf16 rows are copied as is
      } else {
        float f[8];
        unpack(rs.a[c], f);
        const float gv[8] = {rs.gm[0].x, rs.gm[0].y, rs.gm[0].z, rs.gm[0].w,
                             rs.gm[1].x, rs.gm[1].y, rs.gm[1].z, rs.gm[1].w};
        const float bv[8] = {rs.bt[0].x, rs.bt[0].y, rs.bt[0].z, rs.bt[0].w,
                             rs.bt[1].x, rs.bt[1].y, rs.bt[1].z, rs.bt[1].w};
        if (NORM == NORM_LAYER) {
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] = (f[j] - s_a[c]) * s_b[c] * gv[j] + bv[j];
        } else if (NORM == NORM_RMS) {
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] = (f[j] * s_b[c]) * gv[j];
        }
        st_bf16x8(dst, f);
      }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float w[8];
      unpack(rs.b[c], w);
      st_bf16x8(&Bs[buf][srow + RS * c][skc], w);
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  const int fr = lane & 15, fk = (lane >> 4) * 8;
  const int wrow = wm * (BM / TL::WM), wcol = wn * (BN / TL::WN);
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      Frag<bf16> af[TM], bfr[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t) af[t].v = *reinterpret_cast<const bf16x8*>(&As[buf][wrow + t * 16 + fr][ks + fk]);
#pragma unroll
      for (int t = 0; t < TN; ++t) bfr[t].v = *reinterpret_cast<const bf16x8*>(&Bs[buf][wcol + t * 16 + fr][ks + fk]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) mfma_16x16x32(acc[i][j], af[i], bfr[j]);
    }
  };

  const int nk = K / BK;
  load_tiles(rs0, 0);
  store_tiles(rs0, 0);
  if (nk > 1) load_tiles(rs1, BK);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    if (kt + 2 < nk) load_tiles(rs0, (kt + 2) * BK);
    compute(0);
    if (kt + 1 < nk) store_tiles(rs1, 1);
    __syncthreads();
    if (kt + 1 >= nk) break;
    if (kt + 3 < nk) load_tiles(rs1, (kt + 3) * BK);
    compute(1);
    if (kt + 2 < nk) store_tiles(rs0, 0);
    __syncthreads();
  }

  // ---- epilogue: scale/bias/act in registers; TM passes, each staging one 16-row
  // strip per wavefront row (WM*16 rows x BN) through LDS and writing it out as
  // coalesced 8-column chunks (16-byte residual loads and output stores).
  float* Cs = reinterpret_cast<float*>(smem);
  const float* bias = reinterpret_cast<const float*>(g.bias);
  float sc[TN], bi[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wcol + j * 16 + fr;
    sc[j] = (g.w_scale && n < N) ? g.w_scale[n] : 1.0f;
    bi[j] = (bias && n < N) ? bias[n] : 0.0f;
  }
  constexpr int RCH = BN / 8;               // 8-column chunks per output row
  constexpr int PROWS = TL::WM * 16;        // rows staged per pass
  const int res_rows = g.res_rows > 0 ? (int)g.res_rows : M;
  const float* res = reinterpret_cast<const float*>(g.res);
  TOUT* out = reinterpret_cast<TOUT*>(g.out);
  const WtOut store(out, (int64_t)M * g.ld_out * (int64_t)sizeof(TOUT), wt_one_wave());
#pragma unroll
  for (int p = 0; p < TM; ++p) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = acc[p][j][r] * sc[j] + bi[j];
        if (ACT == ACT_GELU) v = sizeof(TOUT) == 2 ? gelu_erf_bf16out(v) : gelu_erf(v);
        Cs[(wm * 16 + (lane >> 4) * 4 + r) * TL::EPI_LD + wcol + j * 16 + fr] = v;
      }
    __syncthreads();
    for (int c = tid; c < PROWS * RCH; c += TL::THREADS) {
      const int lr = c / RCH, cc = (c % RCH) * 8;
      const int m = m0 + (lr >> 4) * (BM / TL::WM) + p * 16 + (lr & 15), n = n0 + cc;
      if (m >= M || n >= N) continue;
      float v[8];
      const float4 a = *reinterpret_cast<const float4*>(&Cs[lr * TL::EPI_LD + cc]);
      const float4 b = *reinterpret_cast<const float4*>(&Cs[lr * TL::EPI_LD + cc + 4]);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      const bool full = n + 8 <= N;
      if (RES) {
        const float* rp = res + (int64_t)(m % res_rows) * g.ld_res + n;
        if (full) {
          const float4 x0 = reinterpret_cast<const float4*>(rp)[0], x1 = reinterpret_cast<const float4*>(rp)[1];
          v[0] += x0.x; v[1] += x0.y; v[2] += x0.z; v[3] += x0.w;
          v[4] += x1.x; v[5] += x1.y; v[6] += x1.z; v[7] += x1.w;
        } else {
          for (int e = 0; e < 8 && n + e < N; ++e) v[e] += rp[e];
        }
      }
      TOUT* op = out + (int64_t)m * g.ld_out + n;
      if (full) {
        if constexpr (sizeof(TOUT) == 2) {
          st_bf16x8_out(reinterpret_cast<bf16*>(op), v, store);
        } else {
          store(reinterpret_cast<float4*>(op), make_float4(v[0], v[1], v[2], v[3]));
          store(reinterpret_cast<float4*>(op) + 1, make_float4(v[4], v[5], v[6], v[7]));
        }
      } else {
        for (int e = 0; e < 8 && n + e < N; ++e) op[e] = from_f32<TOUT>(v[e]);
      }
    }
    __syncthreads();
  }
}

template <class TL, class TX, class TW, int NORM, int ACT, bool RES, class TOUT>
int launch(const GemmArgs& g, hipStream_t stream) {
  const dim3 grid((unsigned)cdiv(g.N, TL::BN), (unsigned)cdiv(g.M, TL::BM));
  hipLaunchKernelGGL((gemm_fast_kernel<TL, TX, TW, NORM, ACT, RES, TOUT>), grid, dim3(TL::THREADS), 0, stream, g);
  CORTEX_CHECK_LAUNCH("gemm_fast_kernel");
  return 1;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Tile configurations (selected per call by the shape heuristic below, or forced
// with CORTEX_GEMM_TILE for tuning sweeps).
using T128x128 = Tile<128, 128, 2, 2, 64>;
using T128x128k32 = Tile<128, 128, 2, 2, 32>;
using T256x128 = Tile<256, 128, 2, 2, 32>;
using T128x256 = Tile<128, 256, 2, 2, 32>;
using T64x128 = Tile<64, 128, 1, 2, 64>;

int forced_tile() {
  static int v = [] {
    const char* s = getenv("CORTEX_GEMM_TILE");
    return s ? atoi(s) : -1;
  }();
  return v;
}

template <class TX, class TW, int NORM, int ACT, bool RES, class TOUT>
int dispatch_tile(const GemmArgs& g, hipStream_t stream) {
  int t = forced_tile();
  if (t < 0) t = 0;
  switch (t) {
    case 1:
      if (g.K % 32 == 0) return launch<T128x128k32, TX, TW, NORM, ACT, RES, TOUT>(g, stream);
      break;
    case 2:
      if (g.K % 32 == 0) return launch<T256x128, TX, TW, NORM, ACT, RES, TOUT>(g, stream);
      break;
    case 3:
      if (g.K % 32 == 0) return launch<T128x256, TX, TW, NORM, ACT, RES, TOUT>(g, stream);
      break;
    case 4:
      if (g.K % 64 == 0) return launch<T64x128, TX, TW, NORM, ACT, RES, TOUT>(g, stream);
      break;
    default:
      break;
  }
  if (g.K % 64 == 0) return launch<T128x128, TX, TW, NORM, ACT, RES, TOUT>(g, stream);
  return launch<T128x128k32, TX, TW, NORM, ACT, RES, TOUT>(g, stream);
}

}  // namespace

int try_gemm_fast(const GemmArgs& g, int x_dtype, int w_dtype, int w_layout, int compute, hipStream_t stream) {
  if (compute != DT_BF16 || w_layout != 0) return 0;
  if (g.K % 32 != 0 || g.M <= 0 || g.N <= 0 || g.M > 0x7fffffff || g.N > 0x7fffffff) return 0;
  const int xs = x_dtype == DT_BF16 ? 2 : 4, ws = w_dtype == DT_I8 ? 1 : 4;
  if (!(x_dtype == DT_BF16 || x_dtype == DT_F32) || !(w_dtype == DT_I8 || w_dtype == DT_F32)) return 0;
  if (!aligned16(g.x) || (g.ld_x * xs) % 16 || !aligned16(g.w) || (g.ld_w * ws) % 16) return 0;
  if (g.norm != NORM_NONE && (g.gamma_dtype != DT_F32 || !aligned16(g.gamma) || (g.beta && !aligned16(g.beta))))
    return 0;
  if (g.bias && g.bias_dtype != DT_F32) return 0;
  const bool res = g.res != nullptr;
  if (res && (g.res_dtype != DT_F32 || g.out_dtype != DT_F32 || !aligned16(g.res) || g.ld_res % 4)) return 0;
  const bool out_bf16 = g.out_dtype == DT_BF16;
  if (!out_bf16 && g.out_dtype != DT_F32) return 0;
  if (!aligned16(g.out) || (g.ld_out * (out_bf16 ? 2 : 4)) % 16) return 0;
  const bool x16 = x_dtype == DT_BF16, w8 = w_dtype == DT_I8;
  // model: LN -> linear (-> GELU) with bf16 output
  if (!x16 && g.norm == NORM_LAYER && !res && out_bf16) {
    if (w8) return g.act ? dispatch_tile<float, int8_t, NORM_LAYER, ACT_GELU, false, bf16>(g, stream)
                         : dispatch_tile<float, int8_t, NORM_LAYER, ACT_NONE, false, bf16>(g, stream);
    return g.act ? dispatch_tile<float, float, NORM_LAYER, ACT_GELU, false, bf16>(g, stream)
                 : dispatch_tile<float, float, NORM_LAYER, ACT_NONE, false, bf16>(g, stream);
  }
  // model: linear + fp32 residual
  if (x16 && g.norm == NORM_NONE && res && !g.act) {
    return w8 ? dispatch_tile<bf16, int8_t, NORM_NONE, ACT_NONE, true, float>(g, stream)
              : dispatch_tile<bf16, float, NORM_NONE, ACT_NONE, true, float>(g, stream);
  }
  // RMSNorm + INT8 linear, bf16 in / out (fused_rmsnorm.norm_linear_int8)
  if (x16 && w8 && g.norm == NORM_RMS && !res && !g.act && out_bf16)
    return dispatch_tile<bf16, int8_t, NORM_RMS, ACT_NONE, false, bf16>(g, stream);
  // QuantizedLinear.forward on bf16 activations
  if (x16 && w8 && g.norm == NORM_NONE && !res && !g.act && out_bf16)
    return dispatch_tile<bf16, int8_t, NORM_NONE, ACT_NONE, false, bf16>(g, stream);
  return 0;
}

}  // namespace cortex
