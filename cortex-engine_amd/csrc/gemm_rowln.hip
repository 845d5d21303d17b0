// Residual linear + the LayerNorm that follows it, in one kernel (gfx950):
//
//   out[m, :] = res[m % res_rows, :] + (A[m, :] . W^T) * w_scale (+ bias)     fp32
//   xn[m, :]  = LN(out[m, :]) * gamma + beta                                   bf16
//               (or, for the opt-in W8A8 mode, int8: clamp(rint(LN(..) / xq_scale), +-127))
// The W8A8 form also takes int8 A rows (A_f = a_scale * A) and the int8 weight (TIN =
// int8_t: v_mfma_i32_16x16x64_i8, exact int32 sums, a_scale * w_scale in the epilogue).
//
// This is SelfAttentionBlock's  x = x + out_proj(attn);  h_in = norm_mlp(x)
// (reference cortex/models/perceiver.py:121-124), and the cross-attention block's
// residual followed by the first self-attention block's norm_attn.  A LayerNorm
// needs whole rows, so a workgroup owns full rows: 32 rows x all N (<= 512) columns,
// 8 wavefronts of 32 x N/8.  With K = 512 the weight (N x K bf16, 512 KiB) is
// re-read by every workgroup from L2, which costs less than a separate LayerNorm
// pass over the fp32 residual stream (read 4 B + write 2 B per element, and a launch).
//
// Operand streaming as in gemm_bf16.hip: direct-to-LDS transfers through a ring of
// STAGES, early stage release, double-buffered fragments, C^T tiles so a lane holds 4
// consecutive columns of one row.  The residual tile is prefetched into registers.
// Row statistics: per wavefront the mean and squared deviations of its columns (lane
// sums, xor-shuffles over the 4 lane groups), combined across the 8 wavefronts through
// LDS in one exchange.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"

namespace cortex {

namespace {

constexpr int RL_BM = 32, RL_BK = 64, RL_WAVES = 8, RL_THREADS = 64 * RL_WAVES;

template <int n>
__device__ __forceinline__ void rl_wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | 0x70 | 0xF00 | ((n >> 4) << 14));
}

// Wait until a ring step's transfers landed when `ahead` later steps (PER transfers
// each, at most S - 1) and X other loads were issued after it.
template <int PER, int S, int X>
__device__ __forceinline__ void rl_wait_ahead(int ahead) {
  if constexpr (S >= 3) {
    if (ahead >= 2) {
      rl_wait_vm<2 * PER + X>();
      return;
    }
  }
  if (ahead >= 1)
    rl_wait_vm<PER + X>();
  else
    rl_wait_vm<X>();
}

__device__ __forceinline__ int rl_swz(int r) { return (r >> 1) & 7; }
// int8 weight rows (64 bytes of K per row and step): the 16-byte chunk c of LDS row r holds
// logical chunk c ^ rl_swz8(r), so the 16 rows of one fragment read fall on distinct
// four-bank groups (the layout gemm_bf16.hip uses for the same rows)
__device__ __forceinline__ int rl_swz8(int r) { return ((r >> 3) ^ (r >> 2)) & 3; }

struct RowLnArgs {
  int64_t M, N, K;
  const void* x;  // bf16 rows (int8 in the W8A8 form)
  int64_t ld_x;
  const void* w;
  int64_t ld_w;
  const float* w_scale;
  const float* bias;
  const float* res;
  int64_t ld_res, res_rows;
  float* out;
  int64_t ld_out;
  const float* gamma;
  const float* beta;
  float eps;
  void* xn;  // bf16, or int8 when Q8
  int64_t ld_xn;
  float xq_inv_scale;  // Q8: 1 / activation scale of the consumer
  float a_scale;       // int8 A rows: A_f = a_scale * A
};

// Epilogue of both forms: scale, bias and residual in fp32, the fp32 rows written, then the
// row statistics and the LayerNorm'd rows.  The wavefront holds column block cb: lane (fr, g4),
// tile (i, j): row m0 + 16 i + fr, columns cb WN + 16 j + 4 g4 .. +3.  Every per-column
// parameter is loaded before the first store, so no wait for them drains stores.  `smem` is
// reused for the statistics exchange (2 KiB) after a barrier; the parts are indexed and
// combined by column block, so which wavefront holds a block does not change any result.
template <int BN, bool Q8, class TIN, class ACC, int TM, int TN>
__device__ __forceinline__ void rowln_epilogue(const RowLnArgs& g, const ACC (&acc)[TM][TN],
                                               const float4 (&rv)[TM][TN], int m0, int cb, unsigned char* smem) {
  constexpr int WN = BN / RL_WAVES;
  const int tid = threadIdx.x, lane = tid & 63;
  const int fr = lane & 15, g4 = lane >> 4;
  const int M = (int)g.M;
  const int wcol = cb * WN;
  // the fp32 residual rows and the normalised rows (bf16, or int8 with Q8), written through
  const WtOut store_x(g.out, g.M * g.ld_out * 4, wt_one_wave());
  const WtOut store_xn(g.xn, g.M * g.ld_xn * (Q8 ? 1 : 2), wt_one_wave());
  float4 scv[TN], biv[TN], gmv[TN], bev[TN];
  // absent scale / bias: load any valid row (gamma) and select the neutral value, so
  // the loads stay unconditional (no branch, no extra wait at its merge)
  const float* sp = g.w_scale ? g.w_scale : g.gamma;
  const float* bp = g.bias ? g.bias : g.gamma;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = wcol + 16 * j + 4 * g4;
    scv[j] = *reinterpret_cast<const float4*>(sp + n);
    biv[j] = *reinterpret_cast<const float4*>(bp + n);
    gmv[j] = *reinterpret_cast<const float4*>(g.gamma + n);
    bev[j] = *reinterpret_cast<const float4*>(g.beta + n);
  }
  rl_wait_vm<0>();
  if (!g.w_scale) {
#pragma unroll
    for (int j = 0; j < TN; ++j) scv[j] = make_float4(1.f, 1.f, 1.f, 1.f);
  }
  if constexpr (sizeof(TIN) == 1) {  // int8 A rows: A_f = a_scale * A
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      scv[j].x *= g.a_scale; scv[j].y *= g.a_scale; scv[j].z *= g.a_scale; scv[j].w *= g.a_scale;
    }
  }
  if (!g.bias) {
#pragma unroll
    for (int j = 0; j < TN; ++j) biv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float v[TM][TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const float4 sc = scv[j], bi = biv[j];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      v[i][j][0] = acc[i][j][0] * sc.x + bi.x + rv[i][j].x;
      v[i][j][1] = acc[i][j][1] * sc.y + bi.y + rv[i][j].y;
      v[i][j][2] = acc[i][j][2] * sc.z + bi.z + rv[i][j].z;
      v[i][j][3] = acc[i][j][3] * sc.w + bi.w + rv[i][j].w;
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + i * 16 + fr;
    if (m < M) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
        store_x(reinterpret_cast<float4*>(g.out + (int64_t)m * g.ld_out + wcol + 16 * j + 4 * g4),
                make_float4(v[i][j][0], v[i][j][1], v[i][j][2], v[i][j][3]));
    }
  }

  // Row statistics with one exchange between the 8 wavefronts: each wavefront takes
  // the mean and the sum of squared deviations (M2) of its WN columns of every row
  // (lane sums, then xor-shuffles over the 4 lane groups), and the 8 equal-sized
  // parts combine as mean = avg(mean_w), M2 = sum(M2_w) + WN * sum((mean_w - mean)^2)
  // (Chan, Golub and LeVeque's pairwise update), as stable as two full passes.
  float2* red = reinterpret_cast<float2*>(smem);  // [RL_WAVES][RL_BM]
  constexpr float inv_wn = 1.0f / (float)WN;
  float mean[TM], rstd[TM];
  __syncthreads();  // every operand read of the LDS is done: it may be reused
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += v[i][j][r];
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float mw = sum * inv_wn;
    float m2 = 0.0f;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float d = v[i][j][r] - mw;
        m2 += d * d;
      }
    m2 += __shfl_xor(m2, 16, 64);
    m2 += __shfl_xor(m2, 32, 64);
    if (g4 == 0) red[cb * RL_BM + i * 16 + fr] = make_float2(mw, m2);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    float2 part[RL_WAVES];
    float msum = 0.0f;
#pragma unroll
    for (int w = 0; w < RL_WAVES; ++w) {
      part[w] = red[w * RL_BM + i * 16 + fr];
      msum += part[w].x;
    }
    const float mu = msum * (1.0f / (float)RL_WAVES);
    float m2 = 0.0f, dev = 0.0f;
#pragma unroll
    for (int w = 0; w < RL_WAVES; ++w) {
      const float d = part[w].x - mu;
      m2 += part[w].y;
      dev += d * d;
    }
    mean[i] = mu;
    rstd[i] = 1.0f / sqrtf(fmaf(dev, (float)WN, m2) * (1.0f / (float)BN) + g.eps);
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = wcol + 16 * j + 4 * g4;
    const float4 gm = gmv[j], be = bev[j];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + i * 16 + fr;
      if (m >= M) continue;
      const float y0 = (v[i][j][0] - mean[i]) * rstd[i] * gm.x + be.x;
      const float y1 = (v[i][j][1] - mean[i]) * rstd[i] * gm.y + be.y;
      const float y2 = (v[i][j][2] - mean[i]) * rstd[i] * gm.z + be.z;
      const float y3 = (v[i][j][3] - mean[i]) * rstd[i] * gm.w + be.w;
      if constexpr (Q8) {
        auto q = [&](float y) {
          return (uint32_t)((int)fminf(fmaxf(rintf(y * g.xq_inv_scale), -127.0f), 127.0f) & 0xff);
        };
        *reinterpret_cast<uint32_t*>(reinterpret_cast<int8_t*>(g.xn) + (int64_t)m * g.ld_xn + n) =
            q(y0) | (q(y1) << 8) | (q(y2) << 16) | (q(y3) << 24);
      } else {
        bf16x4 o;
        o[0] = (bf16)y0;
        o[1] = (bf16)y1;
        o[2] = (bf16)y2;
        o[3] = (bf16)y3;
        store_xn(reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(g.xn) + (int64_t)m * g.ld_xn + n), o);
      }
    }
  }
}

// TW = int8_t with bf16 A rows: the QuantizedLinear int8 weight itself, moved into the LDS ring
// by the same direct-to-LDS transfers as bf16 rows (64 bytes of K per row and step, half the
// bytes, so the ring may hold more stages), and each lane widens its 8-byte fragment exactly
// to bf16 (every int8 value is a bf16 value) right before the MFMAs that use it.
template <int BN, int S, bool Q8 = false, class TIN = bf16, class TW = TIN>
__global__ __launch_bounds__(RL_THREADS) void gemm_rowln_kernel(RowLnArgs g) {
  using OP = Operand<TIN>;
  typedef typename OP::frag frag;
  constexpr int EPC = OP::EPC, BK = 8 * EPC;  // K elements per 16-byte chunk and per 128-byte LDS row
  constexpr int WN = BN / RL_WAVES;   // columns per wavefront
  constexpr int TM = RL_BM / 16, TN = WN / 16;
  constexpr bool WI8 = sizeof(TW) == 1 && sizeof(TIN) == 2;
  constexpr int A_STAGE = RL_BM * 128, W_STAGE = BN * (WI8 ? 64 : 128);  // bytes
  constexpr int WB = W_STAGE / 1024 / RL_WAVES;             // W transfers per wavefront and step
  constexpr int PER = 1 + WB;                                // + one A transfer (blocks shared 2:1)
  constexpr int RING = S * (A_STAGE + W_STAGE);
  static_assert(A_STAGE == 4 * 1024 && W_STAGE % (1024 * RL_WAVES) == 0 && TN >= 1, "shape");
  static_assert(RING <= 160 * 1024, "LDS");
  static_assert(PER * (S - 1) < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[RING];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int fr = lane & 15, g4 = lane >> 4;
  const int M = (int)g.M, K = (int)g.K;
  const int m0 = blockIdx.x * RL_BM;
  const int wcol = wid * WN;

  // transfer sources: A block (wid & 3) = rows 8 (wid & 3) .. +7 (waves 4..7 repeat
  // waves 0..3: identical bytes to identical addresses); W blocks wid * WB + i
  const int ar = (wid & 3) * 8 + (lane >> 3);
  const TIN* a_src = reinterpret_cast<const TIN*>(g.x) + (int64_t)min(m0 + ar, M - 1) * g.ld_x +
                     ((lane & 7) ^ rl_swz(ar)) * EPC;
  const TW* w_src[WB];
  if constexpr (WI8) {
    // lane i of block q writes LDS bytes [16 i, 16 i + 16): row 16 q + i / 4, stored chunk i % 4
#pragma unroll
    for (int i = 0; i < WB; ++i) {
      const int r = (wid * WB + i) * 16 + (lane >> 2);
      w_src[i] = reinterpret_cast<const TW*>(g.w) + (int64_t)r * g.ld_w + ((lane & 3) ^ rl_swz8(r)) * 16;
    }
  } else {
#pragma unroll
    for (int i = 0; i < WB; ++i) {
      const int r = (wid * WB + i) * 8 + (lane >> 3);
      w_src[i] = reinterpret_cast<const TW*>(g.w) + (int64_t)r * g.ld_w + ((lane & 7) ^ rl_swz(r)) * EPC;
    }
  }
  auto a_stage = [&](int s) { return smem + s * A_STAGE; };
  auto w_stage = [&](int s) { return smem + S * A_STAGE + s * W_STAGE; };
  const int nk = K / BK;
  auto issue = [&](int kt) {
    const int s = kt % S, k0 = kt * BK;  // (K elements: bytes for the int8 rows)
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(a_src + k0),
                                     static_cast<void*>(a_stage(s) + (wid & 3) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < WB; ++i)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(w_src[i] + k0),
                                       static_cast<void*>(w_stage(s) + (wid * WB + i) * 1024), 16, 0, 0);
  };

  typename OP::accum acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (typename OP::accum){0, 0, 0, 0};
  int a_off[TM], a_sw[TM], w_off[TN], w_sw[TN];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int r = t * 16 + fr;
    a_off[t] = r * 128;
    a_sw[t] = rl_swz(r);
  }
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int r = wcol + t * 16 + fr;
    w_off[t] = r * (WI8 ? 64 : 128);
    w_sw[t] = WI8 ? rl_swz8(r) : rl_swz(r);
  }
  // W fragments as read from LDS: bf16 fragments, or the raw 8 int8 bytes, widened right
  // before their TM uses
  typedef typename std::conditional<WI8, uint2, frag>::type wfrag;
  auto read_frags = [&](int stage, int ks, frag (&af)[TM], wfrag (&wf)[TN]) {
    const unsigned char* as = a_stage(stage);
    const unsigned char* ws = w_stage(stage);
#pragma unroll
    for (int t = 0; t < TM; ++t)
      af[t] = *reinterpret_cast<const frag*>(as + a_off[t] + (((ks * 4 + g4) ^ a_sw[t]) << 4));
    if constexpr (WI8) {
      // K [32 ks + 8 g4, +8) of the row: logical chunk 2 ks + g4 / 2, half g4 % 2
#pragma unroll
      for (int t = 0; t < TN; ++t)
        wf[t] = *reinterpret_cast<const uint2*>(ws + w_off[t] + (((2 * ks + (g4 >> 1)) ^ w_sw[t]) << 4) +
                                                ((g4 & 1) << 3));
    } else {
#pragma unroll
      for (int t = 0; t < TN; ++t)
        wf[t] = *reinterpret_cast<const frag*>(ws + w_off[t] + (((ks * 4 + g4) ^ w_sw[t]) << 4));
    }
  };
  auto mma = [&](const frag (&af)[TM], const wfrag (&wf)[TN]) {
    if constexpr (WI8) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const frag w = widen_i8x8(wf[j]);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = OP::mma(w, af[i], acc[i][j]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = OP::mma(wf[j], af[i], acc[i][j]);
    }
  };

#pragma unroll
  for (int p = 0; p < S; ++p)
    if (p < nk) issue(p);
  // The residual tile goes into registers right after the first ring stages: the first
  // MFMAs do not wait for it and its latency hides behind the main loop.  Its RV loads
  // sit behind the prologue's transfers in the wave's vmcnt (the scheduling barrier keeps
  // the compiler from moving them in front).
  __builtin_amdgcn_sched_barrier(0);
  const int res_rows = g.res_rows > 0 ? (int)g.res_rows : M;
  float4 rv[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = min(m0 + i * 16 + fr, M - 1);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      rv[i][j] = *reinterpret_cast<const float4*>(g.res + (int64_t)(m % res_rows) * g.ld_res + wcol + 16 * j + 4 * g4);
  }

  constexpr int RV = TM * TN;
  auto wait_step = [&](int j, int last) {  // this wave's transfers of step j landed
    const int ahead = min(nk - 1, last) - j;
    if (j < S)
      rl_wait_ahead<PER, S, RV>(ahead);  // prologue step: the residual loads came after it
    else
      rl_wait_ahead<PER, S, 0>(ahead);
  };
  frag af0[TM], af1[TM];
  wfrag wf0[TN], wf1[TN];
  wait_step(0, S - 1);
  __builtin_amdgcn_s_barrier();
  read_frags(0, 0, af0, wf0);
  // One K step that hands over to the next (as in gemm_bf16.hip): the loop is peeled so that
  // no branch joins in front of an MFMA group, where the compiler would wait for the
  // fragment reads just issued, and each step first waits explicitly for the fragments read
  // after the previous barrier.
  auto step = [&](int kt, auto refill) {
    const int st = kt % S;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): sub-step 0's fragments
    read_frags(st, 1, af1, wf1);
    mma(af0, wf0);
    wait_step(kt + 1, kt + S - 1);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's reads of stage st done
    __builtin_amdgcn_s_barrier();        // all waves done with stage st; step kt+1 visible
    read_frags((kt + 1) % S, 0, af0, wf0);
    if constexpr (decltype(refill)::value) issue(kt + S);
    mma(af1, wf1);
  };
  int kt = 0;
  for (; kt + S < nk; ++kt) step(kt, std::integral_constant<bool, true>{});
  for (; kt + 1 < nk; ++kt) step(kt, std::integral_constant<bool, false>{});
  __builtin_amdgcn_s_waitcnt(0xC07F);  // the last step
  read_frags((nk - 1) % S, 1, af1, wf1);
  mma(af0, wf0);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  mma(af1, wf1);

  rowln_epilogue<BN, Q8, TIN>(g, acc, rv, m0, wid, smem);
}

// Direct-weight form, bf16 A rows and K = 64 * NK (the out-projection shapes), for the weight
// in MFMA fragment order (cortex_frag_weight: 1 KiB blocks of 16 rows x 32 K in lane order).
// The W rows of a wavefront's WN output columns are read by that wavefront alone, so staging
// them in LDS only adds a copy and a barrier per K step.  Here each fragment (t, ks) of K step
// kt is one contiguous 1 KiB read straight into the lane's operand registers (lane (fr, g4):
// row wcol + 16 t + fr, K [64 kt + 32 ks + 8 g4, +8)), RL_DW_AHEAD K steps ahead of its MFMAs,
// with no barrier in the K loop.  (From plain (N, K) rows the same fragment is 64 bytes of 16
// rows, half lines, which measured slower than the LDS ring.)  The 32 A rows, which every
// wavefront reads, move into LDS once before the loop (all of K: 32 * K * 2 bytes, the ring's
// swizzled layout, one 64-deep K step per 4 KiB).  Same fragments and the same accumulation
// order as the ring form, so the results are bit-identical to it.
constexpr int RL_DW_AHEAD = 2;  // 2: forward 0.6945-0.6968 ms; 3: 0.6970-0.6990; 4: 0.6961-0.6986

template <int BN, int NK, bool Q8>
__global__ __launch_bounds__(RL_THREADS) void gemm_rowln_dw_kernel(RowLnArgs g) {
  using OP = Operand<bf16>;
  typedef typename OP::frag frag;
  constexpr int WN = BN / RL_WAVES, TM = RL_BM / 16, TN = WN / 16, WD = RL_DW_AHEAD;
  constexpr int A_STAGE = RL_BM * 128;                   // 32 rows x 64 K of bf16
  constexpr int AB = NK * (A_STAGE / 1024) / RL_WAVES;   // 1 KiB A transfers per wavefront
  constexpr int RED = RL_WAVES * RL_BM * 8;              // the epilogue's statistics exchange
  constexpr int LDS = NK * A_STAGE > RED ? NK * A_STAGE : RED;
  constexpr int RV = TM * TN, WOPS = TN * 2;             // residual loads; W loads per K step
  static_assert(NK * (A_STAGE / 1024) % RL_WAVES == 0 && NK >= WD && TN >= 1, "shape");
  static_assert(RV + WD * WOPS < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[LDS];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int fr = lane & 15, g4 = lane >> 4;
  const int M = (int)g.M;
  const int m0 = blockIdx.x * RL_BM;
  // column block of this wavefront, rotated by workgroup: at any moment the workgroups of an
  // XCD stream 8 different weight blocks rather than all the same 4 KiB per wavefront index
  // (out-projection at B = 32: 16.34-16.41 -> 16.13-16.20 us, same box)
  const int cb = (wid + (int)blockIdx.x) & (RL_WAVES - 1);
  const int wcol = cb * WN;

  // A: the 1 KiB block q = wid * AB + i holds rows 8 (q % 4) .. +7 of K step q / 4 (lane i of a
  // transfer: row i / 8, stored chunk i % 8 = logical chunk (i % 8) ^ rl_swz(row))
  const bf16* A = reinterpret_cast<const bf16*>(g.x);
#pragma unroll
  for (int i = 0; i < AB; ++i) {
    const int q = wid * AB + i, r = (q & 3) * 8 + (lane >> 3);
    const bf16* src = A + (int64_t)min(m0 + r, M - 1) * g.ld_x + (q >> 2) * 64 + ((lane & 7) ^ rl_swz(r)) * 8;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), static_cast<void*>(smem + q * 1024), 16, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // fragment (t, ks) of K step kt: block (wcol / 16 + t, 2 kt + ks), this lane's 16 bytes
  const bf16* wp = reinterpret_cast<const bf16*>(g.w) + (int64_t)(wcol / 16) * (2 * NK) * 512 + lane * 8;
  frag wb[NK][TN][2];  // (fully unrolled: each K step's fragments are registers of their own)
  auto load_w = [&](int kt) {
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        wb[kt][t][ks] = *reinterpret_cast<const frag*>(wp + (t * (2 * NK) + 2 * kt + ks) * 512);
  };
#pragma unroll
  for (int p = 0; p < WD; ++p) load_w(p);
  // the residual tile after the first W steps, so the first MFMAs do not wait for it
  __builtin_amdgcn_sched_barrier(0);
  const int res_rows = g.res_rows > 0 ? (int)g.res_rows : M;
  float4 rv[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = min(m0 + i * 16 + fr, M - 1);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      rv[i][j] = *reinterpret_cast<const float4*>(g.res + (int64_t)(m % res_rows) * g.ld_res + wcol + 16 * j + 4 * g4);
  }
  __builtin_amdgcn_sched_barrier(0);

  typename OP::accum acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (typename OP::accum){0, 0, 0, 0};
  int a_off[TM], a_sw[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int r = t * 16 + fr;
    a_off[t] = r * 128;
    a_sw[t] = rl_swz(r);
  }
  rl_wait_vm<RV + WD * WOPS>();  // this wave's A transfers landed (the W and residual loads came after)
  __builtin_amdgcn_s_barrier();  // every wave's: all 32 A rows in LDS
#pragma unroll
  for (int kt = 0; kt < NK; ++kt) {
    const unsigned char* as = smem + kt * A_STAGE;
    frag af[2][TM];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[ks][t] = *reinterpret_cast<const frag*>(as + a_off[t] + (((ks * 4 + g4) ^ a_sw[t]) << 4));
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = OP::mma(wb[kt][j][ks], af[ks][i], acc[i][j]);
    if (kt + WD < NK) load_w(kt + WD);
    __builtin_amdgcn_sched_barrier(0);  // a K step's loads stay behind its MFMAs (registers)
  }
  rowln_epilogue<BN, Q8, bf16>(g, acc, rv, m0, cb, smem);
}

bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

}  // namespace cortex

using namespace cortex;

namespace {

int residual_ln(const char* who, int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, const void* w,
                int64_t ld_w, const float* w_scale, const float* bias, const float* res, int64_t ld_res,
                int64_t res_rows, float* out, int64_t ld_out, const float* gamma, const float* beta, float eps,
                void* xn, int64_t ld_xn, float xq_scale, bool q8, hipStream_t stream, float a_scale = 0.0f,
                int w_dtype = DT_BF16) {
  const bool i8in = a_scale > 0.0f;  // int8 A rows and weight (W8A8)
  const bool wi8 = !i8in && w_dtype == DT_I8;  // bf16 rows x the int8 weight (widened in the kernel)
  const bool frag = !i8in && w_dtype == DT_BF16_FRAG;  // bf16 rows x the weight in fragment order
  CORTEX_CHECK_ARG(w_dtype == DT_BF16 || w_dtype == DT_I8 || (!i8in && w_dtype == DT_BF16_FRAG),
                   "%s: weight must be bf16, int8 or bf16 in fragment order (got %d)", who, w_dtype);
  CORTEX_CHECK_ARG(!frag || K == 256 || K == 512, "%s: the fragment-order weight needs K = 256 or 512", who);
  if (frag) ld_w = K;  // (the blocks are dense; only the bounds check below reads it)
  CORTEX_CHECK_ARG(M >= 0 && K > 0, "%s: need M >= 0 and K > 0", who);
  CORTEX_CHECK_ARG(N == 256 || N == 512, "%s: N must be 256 or 512 (got %lld)", who, (long long)N);
  CORTEX_CHECK_ARG(K % (i8in ? 2 * RL_BK : RL_BK) == 0 && K <= 0x7fffffffLL, "%s: K must be a multiple of %d", who,
                   i8in ? 2 * RL_BK : RL_BK);
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(M <= 0x7fffffffLL - RL_BM, "%s: M too large", who);
  CORTEX_CHECK_ARG(x && w && res && out && gamma && beta && xn, "%s: null pointer", who);
  CORTEX_CHECK_ARG(res_rows >= 0, "%s: res_rows must be >= 0", who);
  CORTEX_CHECK_ARG(!q8 || xq_scale > 0.0f, "%s: the int8 scale must be positive", who);
  CORTEX_CHECK_ARG(ld_x >= K && ld_w >= K && ld_res >= N && ld_out >= N && ld_xn >= N, "%s: row strides too small",
                   who);
  CORTEX_CHECK_ARG(a16(x) && a16(w) && a16(res) && a16(out) && a16(xn) && a16(gamma) && a16(beta) &&
                       (!w_scale || a16(w_scale)) && (!bias || a16(bias)) && ld_x % (i8in ? 16 : 8) == 0 &&
                       ld_w % (i8in || wi8 ? 16 : 8) == 0 &&
                       ld_res % 4 == 0 && ld_out % 4 == 0 && ld_xn % (q8 ? 16 : 8) == 0,
                   "%s: operands must be 16-byte aligned rows", who);
  RowLnArgs a{M,     N,     K,     x,   ld_x, w,     ld_w, w_scale, bias, res, ld_res, res_rows, out, ld_out,
              gamma, beta,  eps,   xn,  ld_xn, q8 ? 1.0f / xq_scale : 0.0f, a_scale};
  const dim3 grid((unsigned)cdiv(M, (int64_t)RL_BM));
  if (frag) {  // bf16 rows x the fragment-order weight: the direct-weight form
#define RL_DW(BN_, NK_)                                                                                           \
  do {                                                                                                            \
    if (q8) hipLaunchKernelGGL((gemm_rowln_dw_kernel<BN_, NK_, true>), grid, dim3(RL_THREADS), 0, stream, a);   \
    else hipLaunchKernelGGL((gemm_rowln_dw_kernel<BN_, NK_, false>), grid, dim3(RL_THREADS), 0, stream, a);     \
  } while (0)
    if (N == 512 && K == 512) RL_DW(512, 8);
    else if (N == 512) RL_DW(512, 4);
    else if (K == 512) RL_DW(256, 8);
    else RL_DW(256, 4);
#undef RL_DW
    CORTEX_CHECK_LAUNCH("gemm_rowln_dw_kernel");
    return OK;
  }
  if (i8in) {
    CORTEX_CHECK_ARG(N == 512, "%s: the int8 form needs N = 512", who);
    if (q8)
      hipLaunchKernelGGL((gemm_rowln_kernel<512, 2, true, int8_t>), grid, dim3(RL_THREADS), 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_rowln_kernel<512, 2, false, int8_t>), grid, dim3(RL_THREADS), 0, stream, a);
  } else if (wi8) {
    if (N == 512) {
      if (q8)
        hipLaunchKernelGGL((gemm_rowln_kernel<512, 2, true, bf16, int8_t>), grid, dim3(RL_THREADS), 0, stream, a);
      else
        hipLaunchKernelGGL((gemm_rowln_kernel<512, 2, false, bf16, int8_t>), grid, dim3(RL_THREADS), 0, stream, a);
    } else {
      if (q8)
        hipLaunchKernelGGL((gemm_rowln_kernel<256, 2, true, bf16, int8_t>), grid, dim3(RL_THREADS), 0, stream, a);
      else
        hipLaunchKernelGGL((gemm_rowln_kernel<256, 2, false, bf16, int8_t>), grid, dim3(RL_THREADS), 0, stream, a);
    }
  } else if (N == 512) {
    if (q8)
      hipLaunchKernelGGL((gemm_rowln_kernel<512, 2, true>), grid, dim3(RL_THREADS), 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_rowln_kernel<512, 2>), grid, dim3(RL_THREADS), 0, stream, a);
  } else {
    if (q8)
      hipLaunchKernelGGL((gemm_rowln_kernel<256, 3, true>), grid, dim3(RL_THREADS), 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_rowln_kernel<256, 3>), grid, dim3(RL_THREADS), 0, stream, a);
  }
  CORTEX_CHECK_LAUNCH("gemm_rowln_kernel");
  return OK;
}

}  // namespace

extern "C" int cortex_linear_residual_ln(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, int w_dtype,
                                         const void* w, int64_t ld_w, const float* w_scale, const float* bias,
                                         const float* res, int64_t ld_res, int64_t res_rows, float* out,
                                         int64_t ld_out, const float* gamma, const float* beta, float eps, void* xn,
                                         int64_t ld_xn, hipStream_t stream) {
  return residual_ln("cortex_linear_residual_ln", M, N, K, x, ld_x, w, ld_w, w_scale, bias, res, ld_res, res_rows,
                     out, ld_out, gamma, beta, eps, xn, ld_xn, 0.0f, false, stream, 0.0f, w_dtype);
}

extern "C" int cortex_linear_residual_ln_i8(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x,
                                            int w_dtype, const void* w, int64_t ld_w, const float* w_scale,
                                            const float* bias, const float* res, int64_t ld_res, int64_t res_rows,
                                            float* out, int64_t ld_out, const float* gamma, const float* beta,
                                            float eps, int8_t* xq, int64_t ld_xq, float xq_scale,
                                            hipStream_t stream) {
  return residual_ln("cortex_linear_residual_ln_i8", M, N, K, x, ld_x, w, ld_w, w_scale, bias, res, ld_res,
                     res_rows, out, ld_out, gamma, beta, eps, xq, ld_xq, xq_scale, true, stream, 0.0f, w_dtype);
}

extern "C" int cortex_linear_residual_ln_w8a8(int64_t M, int64_t N, int64_t K, const int8_t* xq, int64_t ld_x,
                                              float a_scale, const int8_t* w, int64_t ld_w, const float* w_scale,
                                              const float* bias, const float* res, int64_t ld_res, int64_t res_rows,
                                              float* out, int64_t ld_out, const float* gamma, const float* beta,
                                              float eps, void* xn, int xn_dtype, float xn_scale, int64_t ld_xn,
                                              hipStream_t stream) {
  const char* who = "cortex_linear_residual_ln_w8a8";
  CORTEX_CHECK_ARG(a_scale > 0.0f, "%s: a_scale must be positive", who);
  CORTEX_CHECK_ARG(xn_dtype == DT_BF16 || xn_dtype == DT_I8, "%s: xn must be bf16 or int8", who);
  return residual_ln(who, M, N, K, xq, ld_x, w, ld_w, w_scale, bias, res, ld_res, res_rows, out, ld_out, gamma, beta,
                     eps, xn, ld_xn, xn_scale, xn_dtype == DT_I8, stream, a_scale);
}
