// Self-attention of one Perceiver block with its QKV projection, fused (gfx950):
//
//   [q | k | v]_h = xn_b . W_{qkv,h}^T * w_scale (+ bias)   (L x 3 Dh, kept in LDS, bf16)
//   o_{b,h}      = softmax(q k^T * scale) v                  (L x Dh -> merged-head rows)
//
// SelfAttentionBlock (reference cortex/models/perceiver.py:113-121): qkv_proj on the
// norm_attn rows, split into heads, SDPA.  One workgroup per (head h, sample b) with
// L <= 256 latents: the projection is the 256 x 192 tile [q_h | k_h | v_h] of the
// qkv GEMM (A = the sample's xn rows, W = the head's 3 x 64 weight rows), computed on
// the MFMAs through the same direct-to-LDS ring as the bf16 GEMM, then written once
// into LDS in the layouts the attention reads -- Q and K rows with chunk swizzles, V
// transposed (the V tiles are computed as C rather than C^T, so a lane holds 4
// consecutive keys of one head dimension) -- and the attention runs on it without
// touching HBM.  The qkv activations (B*L x 3D bf16) are never written or re-read.
//
// Attention as in attention_fast.hip: S^T = K Q^T, lane-local online softmax in the
// exp2 domain with a lazily moved reference max, O^T = V^T P^T, row sums on the MFMA.
//
// The opt-in W8A8 form (TIN = int8_t) projects int8 xn rows (xn_f = a_scale * xn) with the
// int8 qkv weight on v_mfma_i32_16x16x64_i8 (exact int32 sums, a_scale * w_scale in the
// epilogue); the attention itself stays bf16.  With Q8OUT the merged-head output is written
// as int8 at out_proj's activation scale, clamp(rint(o * out_inv_scale), -127, 127).
#include <hip/hip_runtime.h>

#include "common.h"

namespace cortex {

namespace {

constexpr int BA_L = 256;                    // latents per workgroup (max)
constexpr int BA_N = 192;                    // q, k, v columns of one head (3 x 64)
constexpr int BA_BK = 64;
constexpr int BA_WM = 4, BA_WN = 2, BA_WAVES = BA_WM * BA_WN, BA_THREADS = 64 * BA_WAVES;
constexpr int BA_TM = BA_L / BA_WM / 16, BA_TN = BA_N / BA_WN / 16;  // 4 x 6 tiles per wave
constexpr int BA_A_STAGE = BA_L * 128, BA_W_STAGE = BA_N * 128;      // bytes
constexpr int BA_AB = BA_A_STAGE / 1024 / BA_WAVES, BA_WB = BA_W_STAGE / 1024 / BA_WAVES;
constexpr int BA_PER = BA_AB + BA_WB;
constexpr int BA_S = 2;
constexpr int BA_RING = BA_S * (BA_A_STAGE + BA_W_STAGE);
constexpr int BA_VP = 144;                   // bytes per V^T row (64 keys + 16 B pad)
constexpr int BA_VTILE = 64 * BA_VP;
constexpr int BA_Q = 0, BA_K = BA_L * 128, BA_VT = 2 * BA_L * 128;
constexpr int BA_ATT = BA_VT + (BA_L / 64) * BA_VTILE;
constexpr int BA_LDS = BA_RING > BA_ATT ? BA_RING : BA_ATT;
constexpr float BA_RESCALE = 8.0f;
static_assert(BA_A_STAGE % (1024 * BA_WAVES) == 0 && BA_W_STAGE % (1024 * BA_WAVES) == 0, "transfer split");

template <int n>
__device__ __forceinline__ void ba_wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | 0x70 | 0xF00 | ((n >> 4) << 14));
}
__device__ __forceinline__ int ba_swz(int r) { return (r >> 1) & 7; }                    // 16 consecutive rows
__device__ __forceinline__ int ba_kswz(int r) { return ((r >> 1) & 1) | ((r >> 2) & 6); }  // K fragment rows
__device__ __forceinline__ int ba_key_of(int st, int r) { return 32 * (st >> 1) + 8 * (r >> 2) + 4 * (st & 1) + (r & 3); }

struct QkvAttnArgs {
  int64_t B, L, D, H;
  const void* xn;  // (B*L, D) rows, bf16 (int8 in the W8A8 form)
  int64_t ld_x;
  const void* w;   // (3D, D) qkv weight image (the int8 weight in the W8A8 form)
  int64_t ld_w;
  const float* w_scale;  // (3D) or null
  const float* bias;     // (3D) or null
  float scale_log2;
  void* out;  // o[b*L + l, h*64 + d], bf16 (or int8 with Q8OUT)
  int64_t ld_o;
  float a_scale;        // W8A8: xn_f = a_scale * xn
  float out_inv_scale;  // Q8OUT
};

// TW = int8_t with bf16 xn rows: the QuantizedLinear int8 qkv weight itself, loaded 8 bytes
// per lane into registers one step ahead and widened exactly to bf16 into the LDS ring
// before the step's barrier (lane (row r, chunk c): logical chunk c of LDS row r).
template <class TIN = bf16, bool Q8OUT = false, class TW = TIN>
__global__ __launch_bounds__(BA_THREADS) void qkv_attention_kernel(QkvAttnArgs a) {
  using OP = Operand<TIN>;
  typedef typename OP::frag frag;
  constexpr int EPC = OP::EPC, BK = 8 * EPC;  // K elements per 16-byte chunk and per 128-byte LDS row
  constexpr bool WI8 = sizeof(TW) == 1 && sizeof(TIN) == 2;
  constexpr int WL = BA_N / (8 * BA_WAVES);  // 8-byte int8 weight loads per lane and step (int8 weights)
  static_assert(BA_N % (8 * BA_WAVES) == 0, "int8 weight staging shape");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[BA_LDS];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int fr = lane & 15, g4 = lane >> 4;
  // the heads of one sample run on one XCD (shared activation panel in its L2)
  const int nh = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + nh * blockIdx.y, total);
  const int h = id % nh;
  const int64_t b = id / nh;
  const int L = (int)a.L, D = (int)a.D;
  const int64_t row0 = b * a.L;

  // ================= projection: C (L x 192) = xn_b . W_h^T =================
  // wavefront (wm, wn): rows wm * 64 .. +63 and the column tiles 2 j + wn (16 columns
  // each): tiles j < 4 are q (j < 2) or k, tiles j >= 4 are v, for both wn -- the MFMA
  // orientation of a tile is then a compile-time property of j
  const int wm = wid / BA_WN, wn = wid % BA_WN;
  const int wrow = wm * (BA_L / BA_WM);
  auto tcol = [&](int j) { return 16 * (2 * j + wn); };
  const TIN* a_src[BA_AB];
#pragma unroll
  for (int i = 0; i < BA_AB; ++i) {
    const int r = (wid * BA_AB + i) * 8 + (lane >> 3);
    a_src[i] = reinterpret_cast<const TIN*>(a.xn) + (row0 + min(r, L - 1)) * a.ld_x + ((lane & 7) ^ ba_swz(r)) * EPC;
  }
  constexpr int NW = WI8 ? WL : BA_WB;
  const TW* w_src[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    // LDS row: q 0..63, k 64..127, v 128..191
    const int r = WI8 ? (wid * WL + i) * 8 + (lane >> 3) : (wid * BA_WB + i) * 8 + (lane >> 3);
    const int64_t grow = (int64_t)(r >> 6) * D + h * 64 + (r & 63);
    w_src[i] = reinterpret_cast<const TW*>(a.w) + grow * a.ld_w + (WI8 ? (lane & 7) * 8 : ((lane & 7) ^ ba_swz(r)) * EPC);
  }
  auto a_stage = [&](int s) { return smem + s * BA_A_STAGE; };
  auto w_stage = [&](int s) { return smem + BA_S * BA_A_STAGE + s * BA_W_STAGE; };
  const int nk = D / BK;
  uint2 wreg[WI8 ? WL : 1];  // int8 weight rows of the last issued step
  auto issue = [&](int kt) {
    const int s = kt % BA_S, k0 = kt * BK;
    if constexpr (WI8) {
#pragma unroll
      for (int i = 0; i < WL; ++i) wreg[i] = *reinterpret_cast<const uint2*>(w_src[i] + k0);
    }
#pragma unroll
    for (int i = 0; i < BA_AB; ++i)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(a_src[i] + k0),
                                       static_cast<void*>(a_stage(s) + (wid * BA_AB + i) * 1024), 16, 0, 0);
    if constexpr (!WI8) {
#pragma unroll
      for (int i = 0; i < BA_WB; ++i)
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(w_src[i] + k0),
                                         static_cast<void*>(w_stage(s) + (wid * BA_WB + i) * 1024), 16, 0, 0);
    }
  };
  auto commit_w = [&](int s) {  // widen the registers into W stage s
    if constexpr (WI8) {
#pragma unroll
      for (int i = 0; i < WL; ++i) {
        const int r = (wid * WL + i) * 8 + (lane >> 3), c = lane & 7;
        *reinterpret_cast<bf16x8*>(w_stage(s) + r * 128 + ((c ^ ba_swz(r)) << 4)) = widen_i8x8(wreg[i]);
      }
    }
  };
  typename OP::accum acc[BA_TM][BA_TN];
#pragma unroll
  for (int i = 0; i < BA_TM; ++i)
#pragma unroll
    for (int j = 0; j < BA_TN; ++j) acc[i][j] = (typename OP::accum){0, 0, 0, 0};
  int a_off[BA_TM], a_sw[BA_TM], w_off[BA_TN], w_sw[BA_TN];
#pragma unroll
  for (int t = 0; t < BA_TM; ++t) {
    const int r = wrow + t * 16 + fr;
    a_off[t] = r * 128;
    a_sw[t] = ba_swz(r);
  }
#pragma unroll
  for (int t = 0; t < BA_TN; ++t) {
    const int r = tcol(t) + fr;
    w_off[t] = r * 128;
    w_sw[t] = ba_swz(r);
  }
  auto read_frags = [&](int stage, int ks, frag (&af)[BA_TM], frag (&wf)[BA_TN]) {
    const unsigned char* as = a_stage(stage);
    const unsigned char* ws = w_stage(stage);
#pragma unroll
    for (int t = 0; t < BA_TM; ++t)
      af[t] = *reinterpret_cast<const frag*>(as + a_off[t] + (((ks * 4 + g4) ^ a_sw[t]) << 4));
#pragma unroll
    for (int t = 0; t < BA_TN; ++t)
      wf[t] = *reinterpret_cast<const frag*>(ws + w_off[t] + (((ks * 4 + g4) ^ w_sw[t]) << 4));
  };
  // q and k tiles as C^T (a lane holds 4 consecutive head dims of one latent), v tiles
  // as C (4 consecutive latents of one head dim)
  auto mma = [&](const frag (&af)[BA_TM], const frag (&wf)[BA_TN]) {
#pragma unroll
    for (int i = 0; i < BA_TM; ++i)
#pragma unroll
      for (int j = 0; j < BA_TN; ++j) acc[i][j] = j < 4 ? OP::mma(wf[j], af[i], acc[i][j]) : OP::mma(af[i], wf[j], acc[i][j]);
  };
  // Both stages in flight; a stage is refilled as soon as every wave holds its last
  // fragments in registers.  Fragments are double-buffered in registers, so the LDS
  // reads of the next K half overlap the MFMAs.
  frag af0[BA_TM], wf0[BA_TN], af1[BA_TM], wf1[BA_TN];
  if constexpr (WI8) {
    issue(0);
    ba_wait_vm<0>();
    commit_w(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): widened rows in LDS before the barrier
    if (1 < nk) issue(1);
  } else {
#pragma unroll
    for (int p = 0; p < BA_S; ++p)
      if (p < nk) issue(p);
    if (nk > 1)
      ba_wait_vm<BA_PER>();
    else
      ba_wait_vm<0>();
  }
  __builtin_amdgcn_s_barrier();
  read_frags(0, 0, af0, wf0);
  // One K step that hands over to the next (as in gemm_bf16.hip): the loop is peeled so that
  // no branch joins in front of an MFMA group, where the compiler would wait for the
  // fragment reads just issued, and each step first waits explicitly for the fragments read
  // after the previous barrier.
  auto step = [&](int kt, auto refill) {
    const int st = kt % BA_S;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): sub-step 0's fragments
    read_frags(st, 1, af1, wf1);
    mma(af0, wf0);
    ba_wait_vm<0>();                     // step kt+1 landed (two stages: nothing newer in flight)
    commit_w((kt + 1) % BA_S);           // (int8 weights: widened into its W stage)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's reads of stage st (and W stores) are done
    __builtin_amdgcn_s_barrier();        // all waves done with stage st; step kt+1 visible
    read_frags((kt + 1) % BA_S, 0, af0, wf0);
    if constexpr (decltype(refill)::value) issue(kt + BA_S);
    mma(af1, wf1);
  };
  int kt = 0;
  for (; kt + BA_S < nk; ++kt) step(kt, std::integral_constant<bool, true>{});
  for (; kt + 1 < nk; ++kt) step(kt, std::integral_constant<bool, false>{});
  __builtin_amdgcn_s_waitcnt(0xC07F);  // the last step
  read_frags((nk - 1) % BA_S, 1, af1, wf1);
  mma(af0, wf0);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  mma(af1, wf1);

  // ---- scale / bias per column, round to bf16, write Q, K rows and V^T into LDS
  float4 scv[BA_TN], biv[BA_TN];  // C^T tiles: 4 consecutive columns
  float scs[BA_TN], bis[BA_TN];   // C tiles: one column per lane
#pragma unroll
  for (int j = 0; j < BA_TN; ++j) {
    const int c = tcol(j);  // first LDS column of the tile
    const int64_t gc = (int64_t)(c >> 6) * D + h * 64 + (c & 63);
    scv[j] = a.w_scale ? *reinterpret_cast<const float4*>(a.w_scale + gc + 4 * g4) : make_float4(1.f, 1.f, 1.f, 1.f);
    biv[j] = a.bias ? *reinterpret_cast<const float4*>(a.bias + gc + 4 * g4) : make_float4(0.f, 0.f, 0.f, 0.f);
    scs[j] = a.w_scale ? a.w_scale[gc + fr] : 1.0f;
    if constexpr (sizeof(TIN) == 1) {  // int8 activations: xn_f = a_scale * xn
      scv[j].x *= a.a_scale; scv[j].y *= a.a_scale; scv[j].z *= a.a_scale; scv[j].w *= a.a_scale;
      scs[j] *= a.a_scale;
    }
    bis[j] = a.bias ? a.bias[gc + fr] : 0.0f;
  }
  __syncthreads();  // every ring read is done: the LDS becomes Q | K | V^T
#pragma unroll
  for (int j = 0; j < BA_TN; ++j) {
    const int c = tcol(j);
    if (j < 4) {  // q or k: rows wrow + 16 i + fr, columns c + 4 g4 .. +3
      const int d = (c & 63) + 4 * g4;
#pragma unroll
      for (int i = 0; i < BA_TM; ++i) {
        const int m = wrow + 16 * i + fr;
        bf16x4 o;
        o[0] = (bf16)(acc[i][j][0] * scv[j].x + biv[j].x);
        o[1] = (bf16)(acc[i][j][1] * scv[j].y + biv[j].y);
        o[2] = (bf16)(acc[i][j][2] * scv[j].z + biv[j].z);
        o[3] = (bf16)(acc[i][j][3] * scv[j].w + biv[j].w);
        const int sw = c < 64 ? ba_swz(m) : ba_kswz(m);
        unsigned char* base = smem + (c < 64 ? BA_Q : BA_K) + m * 128;
        *reinterpret_cast<bf16x4*>(base + (((d >> 3) ^ sw) << 4) + (d & 7) * 2) = o;
      }
    } else {  // v: latents wrow + 16 i + 4 g4 .. +3, head dim (c - 128) + fr
      const int d = (c - 128) + fr;
#pragma unroll
      for (int i = 0; i < BA_TM; ++i) {
        const int m = wrow + 16 * i + 4 * g4;
        bf16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (bf16)(acc[i][j][r] * scs[j] + bis[j]);
        *reinterpret_cast<bf16x4*>(smem + BA_VT + (m >> 6) * BA_VTILE + d * BA_VP + (m & 63) * 2) = o;
      }
    }
  }
  __syncthreads();

  // ================= attention: 32 queries per wavefront =================
  constexpr int QG = 2;
  const int q0 = wid * 16 * QG;
  bf16x8 qf[QG][2];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    const int q = q0 + 16 * qg + fr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qf[qg][ks] = *reinterpret_cast<const bf16x8*>(smem + BA_Q + q * 128 + (((ks * 4 + g4) ^ ba_swz(q)) << 4));
  }
  int k_off[4][2], v_off[2][4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int r = ba_key_of(st, fr);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) k_off[st][ks] = r * 128 + (((ks * 4 + g4) ^ ba_kswz(r)) << 4);
  }
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 4; ++t) v_off[c][t] = (16 * t + fr) * BA_VP + (4 * c + g4) * 16;

  float m_run[QG];
  f32x4 o_acc[QG][4], l_acc[QG];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    m_run[qg] = -INFINITY;
    l_acc[qg] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t) o_acc[qg][t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  }
  bf16x8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = (bf16)1.0f;
  const float sl = a.scale_log2;
  const int nt = (L + 63) / 64;
  // fully unrolled over the (at most 4) key tiles, so one tile's fragment reads and
  // score MFMAs can be scheduled under the previous tile's softmax
#pragma unroll
  for (int kt = 0; kt < BA_L / 64; ++kt) {
    if (kt >= nt) break;
    const unsigned char* ks_ = smem + BA_K + kt * 64 * 128;
    const unsigned char* vs_ = smem + BA_VT + kt * BA_VTILE;
    f32x4 s[QG][4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bf16x8 k0f = *reinterpret_cast<const bf16x8*>(ks_ + k_off[st][0]);
      const bf16x8 k1f = *reinterpret_cast<const bf16x8*>(ks_ + k_off[st][1]);
#pragma unroll
      for (int qg = 0; qg < QG; ++qg) {
        f32x4 acc2 = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0f, qf[qg][0], acc2, 0, 0, 0);
        s[qg][st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1f, qf[qg][1], acc2, 0, 0, 0);
      }
    }
    const int rem = L - kt * 64;
    if (rem < 64) {  // last, partial tile: keys past L
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (32 * (st >> 1) + 8 * g4 + 4 * (st & 1) + i >= rem) {
#pragma unroll
            for (int qg = 0; qg < QG; ++qg) s[qg][st][i] = -INFINITY;
          }
    }
    bf16x8 pf[QG][2];
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) {
      float mx = s[qg][0][0];
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[qg][st][i]);
      if (__any(mx * sl > m_run[qg] + BA_RESCALE)) {  // wave-uniform; always on the first tile
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_tile = mx * sl;
        if (m_run[qg] == -INFINITY) {
          m_run[qg] = m_tile;
        } else {
          const float m_new = fmaxf(m_run[qg], m_tile);
          const float alpha = __builtin_amdgcn_exp2f(m_run[qg] - m_new);
          m_run[qg] = m_new;
          l_acc[qg] *= alpha;
#pragma unroll
          for (int t = 0; t < 4; ++t) o_acc[qg][t] *= alpha;
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[qg][c][i] = (bf16)__builtin_amdgcn_exp2f(fmaf(s[qg][2 * c][i], sl, -m_run[qg]));
          pf[qg][c][4 + i] = (bf16)__builtin_amdgcn_exp2f(fmaf(s[qg][2 * c + 1][i], sl, -m_run[qg]));
        }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int qg = 0; qg < QG; ++qg)
        l_acc[qg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[qg][c], l_acc[qg], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vs_ + v_off[c][t]);
#pragma unroll
        for (int qg = 0; qg < QG; ++qg)
          o_acc[qg][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[qg][c], o_acc[qg][t], 0, 0, 0);
      }
    }
  }
  const WtOut store(a.out, a.B * a.L * a.ld_o * (Q8OUT ? 1 : 2), wt_one_wave());
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    const float l = l_acc[qg][0];
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int q = q0 + 16 * qg + fr;
    if (q < L) {
      if constexpr (Q8OUT) {
        int8_t* O = reinterpret_cast<int8_t*>(a.out) + (row0 + q) * a.ld_o + h * 64;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint32_t pk = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float y = o_acc[qg][t][i] * inv;
            pk |= (uint32_t)((int)fminf(fmaxf(rintf(y * a.out_inv_scale), -127.0f), 127.0f) & 0xff) << (8 * i);
          }
          store(reinterpret_cast<uint32_t*>(O + 16 * t + 4 * g4), pk);
        }
      } else {
        bf16* O = reinterpret_cast<bf16*>(a.out) + (row0 + q) * a.ld_o + h * 64;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bf16x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = (bf16)(o_acc[qg][t][i] * inv);
          store(reinterpret_cast<bf16x4*>(O + 16 * t + 4 * g4), v);
        }
      }
    }
  }
}

bool ba_al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

}  // namespace cortex

using namespace cortex;

extern "C" int cortex_qkv_attention(int64_t B, int64_t L, int64_t D, int64_t H, const void* xn, int64_t ld_x,
                                    int w_dtype, const void* w, int64_t ld_w, const float* w_scale, const float* bias,
                                    float scale, void* out, int64_t ld_o, hipStream_t stream) {
  CORTEX_CHECK_ARG(B >= 0 && L >= 1 && L <= BA_L, "cortex_qkv_attention: need 1 <= L <= %d", BA_L);
  CORTEX_CHECK_ARG(H >= 1 && D == 64 * H && D % BA_BK == 0, "cortex_qkv_attention: need D = 64 * H");
  CORTEX_CHECK_ARG(w_dtype == DT_BF16 || w_dtype == DT_I8, "cortex_qkv_attention: weight must be bf16 or int8");
  if (B == 0) return OK;
  const bool wi8 = w_dtype == DT_I8;
  CORTEX_CHECK_ARG(xn && w && out, "cortex_qkv_attention: null pointer");
  CORTEX_CHECK_ARG(ld_x >= D && ld_w >= D && ld_o >= D, "cortex_qkv_attention: row strides too small");
  CORTEX_CHECK_ARG(ba_al16(xn) && ba_al16(w) && ld_x % 8 == 0 && ld_w % (wi8 ? 16 : 8) == 0 &&
                       ((uintptr_t)out & 7) == 0 && ld_o % 4 == 0 && (!w_scale || ba_al16(w_scale)) &&
                       (!bias || ba_al16(bias)),
                   "cortex_qkv_attention: operands must be 16-byte aligned rows");
  CORTEX_CHECK_ARG(scale > 0.0f && scale < INFINITY, "cortex_qkv_attention: scale must be positive");
  CORTEX_CHECK_ARG(B * H <= 0x7fffffffLL && B <= 65535 && H <= 65535, "cortex_qkv_attention: grid too large");
  QkvAttnArgs a{B, L, D, H, xn, ld_x, w, ld_w, w_scale, bias, scale * 1.4426950408889634f, out, ld_o, 1.0f, 0.0f};
  if (wi8)
    hipLaunchKernelGGL((qkv_attention_kernel<bf16, false, int8_t>), dim3((unsigned)H, (unsigned)B), dim3(BA_THREADS),
                       0, stream, a);
  else
    hipLaunchKernelGGL((qkv_attention_kernel<bf16, false>), dim3((unsigned)H, (unsigned)B), dim3(BA_THREADS), 0,
                       stream, a);
  CORTEX_CHECK_LAUNCH("qkv_attention_kernel");
  return OK;
}

extern "C" int cortex_qkv_attention_w8a8(int64_t B, int64_t L, int64_t D, int64_t H, const int8_t* xq, int64_t ld_x,
                                         float a_scale, const int8_t* w, int64_t ld_w, const float* w_scale,
                                         const float* bias, float scale, void* out, int out_dtype, float out_scale,
                                         int64_t ld_o, hipStream_t stream) {
  const char* who = "cortex_qkv_attention_w8a8";
  CORTEX_CHECK_ARG(B >= 0 && L >= 1 && L <= BA_L, "%s: need 1 <= L <= %d", who, BA_L);
  CORTEX_CHECK_ARG(H >= 1 && D == 64 * H && D % 128 == 0, "%s: need D = 64 * H, a multiple of 128", who);
  CORTEX_CHECK_ARG(out_dtype == DT_BF16 || out_dtype == DT_I8, "%s: out must be bf16 or int8", who);
  if (B == 0) return OK;
  CORTEX_CHECK_ARG(xq && w && out, "%s: null pointer", who);
  CORTEX_CHECK_ARG(a_scale > 0.0f && (out_dtype == DT_BF16 || out_scale > 0.0f), "%s: scales must be positive", who);
  CORTEX_CHECK_ARG(ld_x >= D && ld_w >= D && ld_o >= D, "%s: row strides too small", who);
  CORTEX_CHECK_ARG(ba_al16(xq) && ba_al16(w) && ld_x % 16 == 0 && ld_w % 16 == 0 && ((uintptr_t)out & 7) == 0 &&
                       ld_o % 4 == 0 && (!w_scale || ba_al16(w_scale)) && (!bias || ba_al16(bias)),
                   "%s: operands must be 16-byte aligned rows", who);
  CORTEX_CHECK_ARG(scale > 0.0f && scale < INFINITY, "%s: scale must be positive", who);
  CORTEX_CHECK_ARG(B * H <= 0x7fffffffLL && B <= 65535 && H <= 65535, "%s: grid too large", who);
  QkvAttnArgs a{B, L, D, H, xq, ld_x, w, ld_w, w_scale, bias, scale * 1.4426950408889634f, out, ld_o, a_scale,
                out_dtype == DT_I8 ? 1.0f / out_scale : 0.0f};
  const dim3 grid((unsigned)H, (unsigned)B);
  if (out_dtype == DT_I8)
    hipLaunchKernelGGL((qkv_attention_kernel<int8_t, true>), grid, dim3(BA_THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL((qkv_attention_kernel<int8_t, false>), grid, dim3(BA_THREADS), 0, stream, a);
  CORTEX_CHECK_LAUNCH("qkv_attention_kernel (int8)");
  return OK;
}
