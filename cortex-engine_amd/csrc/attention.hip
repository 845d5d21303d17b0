// Scaled dot-product attention for gfx950 with online softmax over key tiles.
//
// One kernel serves every attention on the Cortex path:
//   * Perceiver cross-attention: batch-invariant latent queries (q batch stride 0)
//     against the sample's ragged events read straight from the CSR key/value
//     buffer (kv_off), so padded event tiles are never visited
//     (reference cortex/models/perceiver.py:75-80 masks them instead);
//   * the reference's block-sparse kernel API: a (n_q, n_k) or (B, n_q, n_k) tile
//     mask with arbitrary BLOCK_L/BLOCK_E, tiles with no allowed element skipped,
//     rows with no allowed key written as 0 (reference sparse_xattn.py:291-328);
//   * per-key padding masks (B, Lk) bool (perceiver.py:75-80 semantics);
//   * self-attention (L = 256) and the behaviour head (Lq = 2).
//
// Layout of the math.  Each wavefront owns 16 queries.  Scores are computed
// transposed, S^T = K Q^T, so that a lane holds the scores of ONE query (lane%16)
// for four keys per 16-key sub-tile; the probabilities P^T are then directly the
// B operand of O^T = V^T P^T (K order permuted identically on both operands), and
// the output accumulator O^T also keeps the query on lane%16.  Row max, row sum
// and the online-softmax rescale are therefore lane-local apart from one
// reduction over the four lane groups (xor 16, xor 32).
// exp is evaluated as exp2 on log2(e)-prescaled scores (FlashAttention-2 style,
// Dao 2023).
#include <hip/hip_runtime.h>

#include "attention.h"
#include "common.h"

namespace cortex {


constexpr int ATT_KT = 64;       // keys per tile
constexpr int ATT_QW = 16;       // queries per wavefront
constexpr int ATT_THREADS = 256; // 4 wavefronts -> 64 queries per workgroup

template <class T>
struct AttnPad;
template <>
struct AttnPad<bf16> {
  static constexpr int P = 8;
};
template <>
struct AttnPad<float> {
  static constexpr int P = 4;
};

template <class T>
__device__ __forceinline__ void load8_any(T (&r)[8], const T* p, int valid, bool vec) {
  if (valid == 8 && vec) {
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(r) = *reinterpret_cast<const uint4*>(p);
    } else {
      reinterpret_cast<uint4*>(r)[0] = reinterpret_cast<const uint4*>(p)[0];
      reinterpret_cast<uint4*>(r)[1] = reinterpret_cast<const uint4*>(p)[1];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (j < valid) ? p[j] : T(0);
  }
}

template <class T>
__device__ __forceinline__ Frag<T> make_frag(const float (&f)[8]) {
  Frag<T> r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r.v[j] = from_f32<T>(f[j]);
  return r;
}

template <class T>
__device__ __forceinline__ Frag<T> frag_from(const T (&x)[8]) {
  Frag<T> r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r.v[j] = x[j];
  return r;
}

template <class T, int DH>
__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(AttnArgs a) {
  constexpr int PAD = AttnPad<T>::P;
  constexpr int KS = DH / 32;   // 32-wide K steps of the score product
  constexpr int DT = DH / 16;   // 16-wide dh tiles of the output
  __shared__ __attribute__((aligned(16))) T Ks[ATT_KT][DH + PAD];
  __shared__ __attribute__((aligned(16))) T Vt[DH][ATT_KT + PAD];
  __shared__ uint8_t kallow[ATT_KT];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g = lane >> 4, fr = lane & 15;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t qb0 = (int64_t)blockIdx.x * (ATT_QW * 4);
  const int64_t q_lane = qb0 + wid * ATT_QW + fr;  // this lane's query
  const bool vec = a.vec != 0;

  // key range of this sample
  int64_t len = a.Lk;
  const T* Kb;
  const T* Vb;
  if (a.kv_off) {
    // offsets come from the caller: clamp them to the Lk key rows of the view
    const int64_t r0 = min(max(a.kv_off[b], (int64_t)0), a.Lk);
    len = min(max(a.kv_off[b + 1], r0), a.Lk) - r0;
    Kb = reinterpret_cast<const T*>(a.k) + r0 * a.k_sl + h * a.k_sh;
    Vb = reinterpret_cast<const T*>(a.v) + r0 * a.v_sl + h * a.v_sh;
  } else {
    Kb = reinterpret_cast<const T*>(a.k) + b * a.k_sb + h * a.k_sh;
    Vb = reinterpret_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh;
  }
  if (a.kv_len) len = min(len, a.kv_len[b]);
  if (len < 0) len = 0;

  // Q fragments (B operand of S^T = K Q^T): query q_lane, dh slice [32ks + 8g, +8)
  Frag<T> qf[KS];
  {
    const T* Qp = reinterpret_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh + q_lane * a.q_sl;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int64_t d = ks * 32 + g * 8;
      const int valid = (q_lane < a.Lq) ? (int)max<int64_t>(0, min<int64_t>(8, a.Dh - d)) : 0;
      T r[8];
      load8_any(r, Qp + (valid > 0 ? d : 0), valid, vec);
      qf[ks] = frag_from<T>(r);
    }
  }

  float m_run = -INFINITY;  // running max (log2 domain) of query q_lane
  float l_run = 0.0f;       // this lane's partial exp-sum (keys of its lane group)
  f32x4 o_acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o_acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  const bool has_bm = a.block_mask != nullptr;
  const uint8_t* bm = has_bm ? a.block_mask + b * a.bm_sb : nullptr;
  const int64_t n_tiles = cdiv(len, ATT_KT);
  for (int64_t kt = 0; kt < n_tiles; ++kt) {
    const int64_t k0 = kt * ATT_KT;
    // which keys of this tile are allowed (padding / key mask), and tile skip test
    int any = 0;
    if (tid < ATT_KT) {
      const int64_t j = k0 + tid;
      uint8_t ok = j < len;
      if (ok && a.key_mask) ok = a.key_mask[b * a.km_sb + j] != 0;
      kallow[tid] = ok;
      any = ok;
    }
    if (has_bm) {
      // any allowed (q-tile, k-tile) pair spanned by this workgroup's queries and tile
      const int64_t qi0 = qb0 / a.block_l, qi1 = min(a.Lq - 1, qb0 + 63) / a.block_l;
      const int64_t kj0 = k0 / a.block_e, kj1 = min(len - 1, k0 + ATT_KT - 1) / a.block_e;
      const int64_t nq = qi1 - qi0 + 1, nk = kj1 - kj0 + 1;
      int anyb = 0;
      for (int64_t p = tid; p < nq * nk; p += ATT_THREADS) {
        const int64_t qi = qi0 + p / nk, kj = kj0 + p % nk;
        if (qi < a.n_qt && kj < a.n_kt && bm[qi * a.n_kt + kj]) anyb = 1;
      }
      anyb = __syncthreads_or(anyb);
      any = __syncthreads_or(any) && anyb;
    } else {
      any = __syncthreads_or(any);
    }
    if (!any) continue;

    // stage K [key][dh] and V^T [dh][key]
    constexpr int DCH = DH / 8;
    for (int c = tid; c < ATT_KT * DCH; c += ATT_THREADS) {
      const int kk = c / DCH, d0 = (c % DCH) * 8;
      const int64_t j = k0 + kk;
      const int valid = (j < len) ? (int)max<int64_t>(0, min<int64_t>(8, a.Dh - d0)) : 0;
      T kr[8], vr[8];
      load8_any(kr, Kb + (valid > 0 ? j * a.k_sl + d0 : 0), valid, vec);
      load8_any(vr, Vb + (valid > 0 ? j * a.v_sl + d0 : 0), valid, vec);
#pragma unroll
      for (int e = 0; e < 8; ++e) Ks[kk][d0 + e] = kr[e];
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[d0 + e][kk] = vr[e];
    }
    __syncthreads();

    // S^T for 4 sub-tiles of 16 keys
    f32x4 s[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      s[st] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        Frag<T> kf;
        const T* src = &Ks[st * 16 + fr][ks * 32 + g * 8];
#pragma unroll
        for (int e = 0; e < 8; ++e) kf.v[e] = src[e];
        mfma_16x16x32(s[st], kf, qf[ks]);
      }
    }
    // mask + scale into the log2 domain; tile max
    float tmax = -INFINITY;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = st * 16 + g * 4 + i;
        bool ok = kallow[kk] != 0;
        if (ok && has_bm) {
          const int64_t qi = q_lane / a.block_l, kj = (k0 + kk) / a.block_e;
          ok = (qi < a.n_qt && kj < a.n_kt) ? (bm[qi * a.n_kt + kj] != 0) : false;
        }
        const float x = ok ? s[st][i] * a.scale_log2 : -INFINITY;
        s[st][i] = x;
        tmax = fmaxf(tmax, x);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    if (m_new != -INFINITY) {
      const float alpha = exp2f(m_run - m_new);  // m_run = -inf -> 0
      float psum = 0.0f;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = exp2f(s[st][i] - m_new);  // masked -> 0
          s[st][i] = p;
          psum += p;
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int t = 0; t < DT; ++t) o_acc[t] *= alpha;
      // O^T += V^T P^T over two 32-key halves
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float pf[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[i] = s[2 * c][i];
          pf[4 + i] = s[2 * c + 1][i];
        }
        const Frag<T> pfrag = make_frag<T>(pf);
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          Frag<T> vf;
          const T* v0 = &Vt[t * 16 + fr][c * 32 + g * 4];
          const T* v1 = &Vt[t * 16 + fr][c * 32 + 16 + g * 4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf.v[e] = v0[e];
            vf.v[4 + e] = v1[e];
          }
          mfma_16x16x32(o_acc[t], vf, pfrag);
        }
      }
      m_run = m_new;
    }
    __syncthreads();  // before the next tile overwrites Ks / Vt / kallow
  }

  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (q_lane < a.Lq) {
    T* O = reinterpret_cast<T*>(a.out) + b * a.o_sb + h * a.o_sh + q_lane * a.o_sl;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t d = t * 16 + g * 4 + i;
        if (d < a.Dh) O[d] = from_f32<T>(o_acc[t][i] * inv);
      }
  }
}

}  // namespace cortex

using namespace cortex;

template <class T>
static int launch_attn(const AttnArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)cdiv(a.Lq, ATT_QW * 4), (unsigned)(a.B * a.H));
  if (a.Dh <= 32)
    hipLaunchKernelGGL((attention_kernel<T, 32>), grid, dim3(ATT_THREADS), 0, stream, a);
  else if (a.Dh <= 64)
    hipLaunchKernelGGL((attention_kernel<T, 64>), grid, dim3(ATT_THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL((attention_kernel<T, 128>), grid, dim3(ATT_THREADS), 0, stream, a);
  CORTEX_CHECK_LAUNCH("attention_kernel");
  return OK;
}

extern "C" int cortex_attention(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dh, const void* q,
                                int64_t q_sb, int64_t q_sh, int64_t q_sl, const void* k, int64_t k_sb, int64_t k_sh,
                                int64_t k_sl, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sl,
                                const int64_t* kv_offsets, const int64_t* kv_lengths, const uint8_t* key_mask,
                                int64_t km_sb, const uint8_t* block_mask, int64_t bm_sb, int64_t n_qt, int64_t n_kt,
                                int64_t block_l, int64_t block_e, float scale, void* out, int64_t o_sb, int64_t o_sh,
                                int64_t o_sl, hipStream_t stream) {
  CORTEX_CHECK_ARG(B >= 0 && H >= 0 && Lq >= 0 && Lk >= 0, "cortex_attention: negative shape");
  if (B == 0 || H == 0 || Lq == 0) return OK;
  CORTEX_CHECK_ARG(Dh >= 1 && Dh <= 128, "cortex_attention: head dim %lld outside [1, 128]", (long long)Dh);
  CORTEX_CHECK_ARG(q && k && v && out, "cortex_attention: null q, k, v or out");
  CORTEX_CHECK_ARG(block_mask == nullptr || (block_l > 0 && block_e > 0 && n_qt > 0 && n_kt > 0),
                   "cortex_attention: block mask needs positive tile sizes and counts");
  CORTEX_CHECK_ARG(B * H <= 65535 && cdiv(Lq, 64) <= 0x7fffffffLL, "cortex_attention: grid too large (B*H=%lld)",
                   (long long)(B * H));
  AttnArgs a = {};
  a.B = B;
  a.H = H;
  a.Lq = Lq;
  a.Lk = Lk;
  a.Dh = Dh;
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sl = q_sl;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_sl = k_sl;
  a.v = v;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sl = v_sl;
  a.kv_off = kv_offsets;
  a.kv_len = kv_lengths;
  a.key_mask = key_mask;
  a.km_sb = km_sb;
  a.block_mask = block_mask;
  a.bm_sb = bm_sb;
  a.n_qt = n_qt;
  a.n_kt = n_kt;
  a.block_l = block_l;
  a.block_e = block_e;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = out;
  a.o_sb = o_sb;
  a.o_sh = o_sh;
  a.o_sl = o_sl;
  const int es = dtype == DT_BF16 ? 2 : 4;
  bool vec = true;
  for (const void* p : {q, k, v}) vec = vec && ((uintptr_t)p % 16 == 0);
  for (int64_t s : {q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl}) vec = vec && ((s * es) % 16 == 0);
  a.vec = vec ? 1 : 0;
  const int fast = try_attention_fast(a, dtype, stream);
  if (fast != 0) return fast > 0 ? OK : fast;
  if (dtype == DT_BF16) return launch_attn<bf16>(a, stream);
  if (dtype == DT_F32) return launch_attn<float>(a, stream);
  set_error("cortex_attention: unsupported dtype %d (bf16 or f32)", dtype);
  return E_UNSUPPORTED;
}
