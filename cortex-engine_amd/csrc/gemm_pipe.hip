// Pipelined bf16 x int8 GEMM for gfx950: direct-to-LDS operand streaming.
//
//   C[m, n] = epi( sum_k A[m, k] * W[n, k] ),  A bf16 (M, K) rows, W int8 (N, K) rows
//   epi: * w_scale[n] (+ bias[n]) (-> erf-GELU) -> bf16, or (+ fp32 residual) -> fp32
//
// Both operands travel HBM/L2 -> LDS with global_load_lds_dwordx4 (16 bytes per lane,
// no VGPRs held while in flight) through a STAGES-deep ring, so the loads of K steps
// j+1 .. j+STAGES-1 are in flight while step j is multiplied.  Synchronisation is an
// explicit vmcnt wait on the wave's own transfers plus a raw s_barrier (a fenced
// __syncthreads would drain every outstanding transfer at each step).
//
// LDS layouts (one K step = 64 columns):
//   A stage: [BM rows][128 B], the 16-byte chunk c of row r stored at chunk c ^ (r & 7)
//            so that the 16 rows read by one MFMA fragment hit distinct banks;
//   W stage: [BN rows][64 B] raw int8, chunk c of row r at chunk c ^ (r & 3).
// A transfer instruction writes 1 KiB contiguous (64 lanes x 16 B); each lane picks
// the global chunk that belongs at its LDS position, which is how the swizzle is made.
// W fragments are widened int8 -> bf16 in registers after the LDS read (exact).
#include <hip/hip_runtime.h>

#include "common.h"
#include "gemm.h"

namespace cortex {

namespace {

// s_waitcnt immediate for "at most n vector-memory operations outstanding"
// (gfx9 encoding: vmcnt[3:0] at bits 3:0, vmcnt[5:4] at bits 15:14, expcnt/lgkmcnt untouched).
template <int n>
__device__ __forceinline__ void wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | 0x70 | 0xF00 | ((n >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

__device__ __forceinline__ void dma16(const void* g, void* lds_block) {
  __builtin_amdgcn_global_load_lds(g, lds_block, 16, 0, 0);
}

// output row chunk of 8 values (global memory only; written through as `store` says)
__device__ __forceinline__ void st_bf16x8(bf16* dst, const float (&f)[8], const WtOut& store) {
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (bf16)f[j];
  store(reinterpret_cast<bf16x8*>(dst), v);
}

template <int BM_, int BN_, int WM_, int WN_, int STAGES_, int WBYTES_ = 1>
struct PTile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, STAGES = STAGES_, BK = 64;
  static constexpr int WBYTES = WBYTES_;  // bytes per weight element: 1 int8, 2 bf16
  static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES;
  static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  static constexpr int A_STAGE = BM * 128, W_STAGE = BN * 64 * WBYTES;  // bytes
  static constexpr int A_BLOCKS = A_STAGE / 1024 / WAVES;           // 1 KiB transfers per wave
  static constexpr int W_BLOCKS = W_STAGE / 1024 / WAVES;
  static constexpr int PER_STEP = A_BLOCKS + W_BLOCKS;              // transfers per wave per K step
  static constexpr int EPI_LD = BN + 4;
  static constexpr int EPI_BYTES = WM * 16 * EPI_LD * 4;
  static constexpr int RING_BYTES = STAGES * (A_STAGE + W_STAGE);
  static constexpr int LDS_BYTES = RING_BYTES > EPI_BYTES ? RING_BYTES : EPI_BYTES;
  static_assert(A_STAGE % (1024 * WAVES) == 0 && W_STAGE % (1024 * WAVES) == 0, "transfer split");
  static_assert(TM >= 1 && TN >= 1, "wave tile");
};

template <class TL, int ACT, bool RES, class TOUT>
__global__ __launch_bounds__(TL::THREADS, 2) void gemm_pipe_kernel(GemmArgs g) {
  constexpr int BM = TL::BM, BN = TL::BN, TM = TL::TM, TN = TL::TN, S = TL::STAGES;
  constexpr int AB = TL::A_BLOCKS, WB = TL::W_BLOCKS, PER = TL::PER_STEP;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[TL::LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / TL::WN, wn = wid % TL::WN;
  const int nbx = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + nbx * blockIdx.y, total);
  const int m0 = (id / nbx) * BM, n0 = (id % nbx) * BN;
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const bf16* __restrict__ A = reinterpret_cast<const bf16*>(g.x);
  const unsigned char* __restrict__ W = reinterpret_cast<const unsigned char*>(g.w);
  constexpr int WROW = 64 * TL::WBYTES;  // bytes of one weight row per K step

  // Global source of each of this lane's transfers (K offset added per step).
  // A block q (of this wave): rows 8q..8q+7; lane -> row 8q + lane/8, LDS chunk lane%8,
  // which holds logical chunk (lane%8) ^ (row & 7).
  const bf16* a_src[AB];
#pragma unroll
  for (int i = 0; i < AB; ++i) {
    const int q = wid * AB + i;
    const int r = q * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    a_src[i] = A + (int64_t)min(m0 + r, M - 1) * g.ld_x + c * 8;
  }
  // W block q: int8 rows of 64 B (16 rows per KiB, chunk swizzle c ^ (row & 3)) or
  // bf16 rows of 128 B (8 rows per KiB, swizzle c ^ (row & 7) as for A).
  constexpr int WCH = WROW / 16, WRPB = 1024 / WROW;  // chunks per row, rows per block
  const unsigned char* w_src[WB];
#pragma unroll
  for (int i = 0; i < WB; ++i) {
    const int q = wid * WB + i;
    const int r = q * WRPB + lane / WCH;
    const int c = (lane % WCH) ^ (r & (WCH - 1));
    w_src[i] = W + ((int64_t)min(n0 + r, N - 1) * g.ld_w) * TL::WBYTES + c * 16;
  }
  auto a_stage = [&](int s) { return smem + s * TL::A_STAGE; };
  auto w_stage = [&](int s) { return smem + S * TL::A_STAGE + s * TL::W_STAGE; };
  auto issue = [&](int kt) {
    const int s = kt % S;
    const int k0 = kt * TL::BK;
#pragma unroll
    for (int i = 0; i < AB; ++i) dma16(a_src[i] + k0, a_stage(s) + (wid * AB + i) * 1024);
#pragma unroll
    for (int i = 0; i < WB; ++i) dma16(w_src[i] + k0 * TL::WBYTES, w_stage(s) + (wid * WB + i) * 1024);
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  const int fr = lane & 15, g4 = lane >> 4;
  const int wrow = wm * (BM / TL::WM), wcol = wn * (BN / TL::WN);
  const int nk = K / TL::BK;

#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p < nk) issue(p);

  for (int kt = 0; kt < nk; ++kt) {
    // own transfers of step kt complete: at most (steps issued after kt) * PER outstanding
    const int ahead = min(nk - 1, kt + S - 2) - kt;
    if (S >= 3 && ahead >= 1) {
      if (S >= 4 && ahead >= 2)
        wait_vm<2 * PER>();
      else
        wait_vm<PER>();
    } else {
      wait_vm<0>();
    }
    __builtin_amdgcn_s_barrier();  // every wave's step-kt data visible; step kt-1 reads done
    if (kt + S - 1 < nk) issue(kt + S - 1);
    const unsigned char* as = a_stage(kt % S);
    const unsigned char* ws = w_stage(kt % S);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      Frag<bf16> af[TM], bfr[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const int r = wrow + t * 16 + fr;
        const int c = (ks * 4 + g4) ^ (r & 7);
        af[t].v = *reinterpret_cast<const bf16x8*>(as + r * 128 + c * 16);
      }
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int r = wcol + t * 16 + fr;
        if constexpr (TL::WBYTES == 2) {
          const int c = (ks * 4 + g4) ^ (r & 7);
          bfr[t].v = *reinterpret_cast<const bf16x8*>(ws + r * 128 + c * 16);
        } else {
          const int kb = ks * 32 + g4 * 8;  // byte offset of this lane's 8 k-values
          const int c = (kb >> 4) ^ (r & 3);
          const uint2 raw = *reinterpret_cast<const uint2*>(ws + r * 64 + c * 16 + (kb & 8));
          bfr[t].v = widen_i8x8(raw);
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) mfma_16x16x32(acc[i][j], af[i], bfr[j]);
    }
  }
  wait_lgkm0();
  __builtin_amdgcn_s_barrier();  // all fragment reads done before the epilogue reuses LDS

  // ---- epilogue (same scheme as the register-staged kernel): TM passes of one 16-row
  // strip per wavefront row through LDS, written out as coalesced 8-column chunks.
  float* Cs = reinterpret_cast<float*>(smem);
  const float* bias = reinterpret_cast<const float*>(g.bias);
  float sc[TN], bi[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wcol + j * 16 + fr;
    sc[j] = (g.w_scale && n < N) ? g.w_scale[n] : 1.0f;
    bi[j] = (bias && n < N) ? bias[n] : 0.0f;
  }
  constexpr int RCH = BN / 8;
  constexpr int PROWS = TL::WM * 16;
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
        Cs[(wm * 16 + g4 * 4 + r) * TL::EPI_LD + wcol + j * 16 + fr] = v;
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
          st_bf16x8(reinterpret_cast<bf16*>(op), v, store);
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

template <class TL, int ACT, bool RES, class TOUT>
int launch(const GemmArgs& g, hipStream_t stream) {
  const dim3 grid((unsigned)cdiv(g.N, TL::BN), (unsigned)cdiv(g.M, TL::BM));
  if (cdiv(g.M, TL::BM) > 65535 || cdiv(g.N, TL::BN) * cdiv(g.M, TL::BM) > 0x7fffffff) return 0;  // grid limits
  hipLaunchKernelGGL((gemm_pipe_kernel<TL, ACT, RES, TOUT>), grid, dim3(TL::THREADS), 0, stream, g);
  CORTEX_CHECK_LAUNCH("gemm_pipe_kernel");
  return 1;
}

using P128x128s3 = PTile<128, 128, 2, 2, 3>;
using P64x128s3 = PTile<64, 128, 1, 2, 3>;
using Q128x128s2 = PTile<128, 128, 2, 2, 2, 2>;
using Q64x128s3 = PTile<64, 128, 1, 2, 3, 2>;

// int8 weights: small grids (N = 512) get the 64-row tile for twice the workgroups
template <int ACT, bool RES, class TOUT>
int dispatch_i8(const GemmArgs& g, hipStream_t stream) {
  return cdiv(g.M, 128) * cdiv(g.N, 128) < 512 ? launch<P64x128s3, ACT, RES, TOUT>(g, stream)
                                                : launch<P128x128s3, ACT, RES, TOUT>(g, stream);
}

// bf16 weights: residual GEMMs (memory bound) take 64-row tiles, twice the workgroups per CU;
// the others 128 x 128 with two stages (two workgroups per CU)
template <int ACT, bool RES, class TOUT>
int dispatch_bf16(const GemmArgs& g, hipStream_t stream) {
  if constexpr (RES)
    return launch<Q64x128s3, ACT, RES, TOUT>(g, stream);
  else
    return launch<Q128x128s2, ACT, RES, TOUT>(g, stream);
}

template <int ACT, bool RES, class TOUT>
int dispatch(const GemmArgs& g, bool w8, hipStream_t stream) {
  return w8 ? dispatch_i8<ACT, RES, TOUT>(g, stream) : dispatch_bf16<ACT, RES, TOUT>(g, stream);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int try_gemm_pipe(const GemmArgs& g, int x_dtype, int w_dtype, int w_layout, int compute, hipStream_t stream) {
  if (compute != DT_BF16 || w_layout != 0 || x_dtype != DT_BF16 || !(w_dtype == DT_I8 || w_dtype == DT_BF16)) return 0;
  if (g.norm != NORM_NONE || g.K % 64 != 0 || g.M <= 0 || g.N <= 0) return 0;
  if (g.M > 0x7fffffff || g.N > 0x7fffffff || g.K > 0x7fffffff) return 0;
  const bool w8 = w_dtype == DT_I8;
  if (!aligned16(g.x) || (g.ld_x * 2) % 16 || !aligned16(g.w) || (g.ld_w * (w8 ? 1 : 2)) % 16) return 0;
  if (g.bias && g.bias_dtype != DT_F32) return 0;
  const bool res = g.res != nullptr;
  if (res && (g.res_dtype != DT_F32 || g.out_dtype != DT_F32 || !aligned16(g.res) || g.ld_res % 4)) return 0;
  const bool out_bf16 = g.out_dtype == DT_BF16;
  if (!out_bf16 && g.out_dtype != DT_F32) return 0;
  if (!aligned16(g.out) || (g.ld_out * (out_bf16 ? 2 : 4)) % 16) return 0;
  if (res) return g.act ? 0 : dispatch<ACT_NONE, true, float>(g, w8, stream);
  if (out_bf16)
    return g.act ? dispatch<ACT_GELU, false, bf16>(g, w8, stream) : dispatch<ACT_NONE, false, bf16>(g, w8, stream);
  return g.act ? dispatch<ACT_GELU, false, float>(g, w8, stream) : dispatch<ACT_NONE, false, float>(g, w8, stream);
}

}  // namespace cortex
