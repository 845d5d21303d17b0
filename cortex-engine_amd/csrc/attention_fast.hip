// Attention fast path for gfx950: bf16 operands, head dim 64, keys bounded only by
// a per-sample length (dense self-attention, CSR cross-attention, broadcast
// queries).  Every attention of the Cortex forward runs here; per-key padding
// masks, block masks, fp32 and other head dims use the general kernel.
//
// Workgroup: 8 wavefronts x 16 queries of one (sample, head).  Keys are taken in
// chunks of up to 4 tiles of 64: every load of a chunk is issued at once (one
// memory round trip per chunk, not per tile), then its tiles are multiplied with
// no further synchronisation.  Two workgroups share a CU (68 KiB LDS each), so one
// loads while the other multiplies.
//
//   scores  S^T = K Q^T    (A = K rows from LDS, B = Q held in registers): a lane
//           holds 4 keys x 1 query per 16x16 sub-tile, so the softmax statistics of
//           a query are lane-local apart from two xor-shuffles (lane groups);
//   output  O^T += V^T P^T (A = V^T rows from LDS, B = P^T straight from the score
//           accumulators, rounded to bf16);
//   sums    l += 1 P^T     (an all-ones A operand: the key-sum of exactly the bf16
//           probabilities used in O, on the matrix core instead of the VALU).
//
// Key order.  Score sub-tile st, row r holds key 32(st/2) + 8(r/4) + 4(st%2) + r%4,
// so a lane of group g ends up with the 8 CONSECUTIVE keys 32c + 8g .. +7 for
// key step c; V^T is then read as one 16-byte LDS word per fragment.
//
// Staging.  K: global -> LDS by direct transfers (global_load_lds_dwordx4), rows of
// 128 B with the 16-byte chunk c of row r stored at c ^ f(r), f chosen so that the
// 16 rows of one fragment read cover all 16 bank groups.  V: each lane loads 4 head
// dims of a pair of keys, packs (key, key+1) dwords and writes them transposed as
// V^T rows of 64 keys with a 144-byte pitch; the 16 rows read by one fragment, and
// the two rows (8 apart) written by the two half-waves, fall into distinct banks.
//
// Online softmax in the exp2 domain (FlashAttention-2, Dao 2023) with a lazily
// moved reference max; keys past the sample's length are masked in the last tile;
// rows with no key give 0.
#include <hip/hip_runtime.h>

#include "attention.h"
#include "common.h"

namespace cortex {

namespace {

constexpr int AF_KT = 64;                        // keys per tile
constexpr int AF_CH = 4;                         // tiles per chunk
constexpr int AF_WAVES = 8;
constexpr int AF_THREADS = 64 * AF_WAVES;
constexpr int AF_QB = 16 * AF_WAVES;             // 128 queries per workgroup
constexpr int AF_KTILE = AF_KT * 128;            // bytes of one K tile (64 keys x 64 bf16)
constexpr int AF_VP = 144;                       // bytes per V^T row (64 keys + 16 B pad)
constexpr int AF_VTILE = 64 * AF_VP;             // bytes of one V^T tile (64 head dims)
constexpr int AF_LDS = AF_CH * (AF_KTILE + AF_VTILE);
// A query's running max is moved only when a tile raises it by more than this
// (log2 units): the probabilities stay <= 2^8, exact in the fp32 sums, and the
// accumulator rescale is skipped for almost every tile after the first.
constexpr float AF_RESCALE = 8.0f;

// K-tile chunk swizzle: bits 1, 3, 4 of the row.  The 16 rows of one fragment read
// (key_of(st, 0..15)) then cover all 16 (row parity, chunk) bank groups.
__device__ __forceinline__ int kswz(int r) { return ((r >> 1) & 1) | ((r >> 2) & 6); }
__device__ __forceinline__ int key_of(int st, int r) {
  return 32 * (st >> 1) + 8 * (r >> 2) + 4 * (st & 1) + (r & 3);
}

__global__ __launch_bounds__(AF_THREADS) __attribute__((amdgpu_waves_per_eu(4)))
void attention_fast_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[AF_LDS];  // K tiles, then V^T tiles
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;

  // Keep the query blocks of one (sample, head) on one XCD (shared K/V in its L2).
  const int nqb = gridDim.x, total = gridDim.x * gridDim.y;
  int id = blockIdx.x + nqb * blockIdx.y;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  const int64_t bh = id / nqb;
  const int qblk = id % nqb;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t q0 = (int64_t)qblk * AF_QB + wid * 16;

  int64_t len = a.Lk;
  const bf16* Kb;
  const bf16* Vb;
  if (a.kv_off) {
    const int64_t r0 = a.kv_off[b];
    len = a.kv_off[b + 1] - r0;
    Kb = reinterpret_cast<const bf16*>(a.k) + r0 * a.k_sl + h * a.k_sh;
    Vb = reinterpret_cast<const bf16*>(a.v) + r0 * a.v_sl + h * a.v_sh;
  } else {
    Kb = reinterpret_cast<const bf16*>(a.k) + b * a.k_sb + h * a.k_sh;
    Vb = reinterpret_cast<const bf16*>(a.v) + b * a.v_sb + h * a.v_sh;
  }
  if (a.kv_len) len = min(len, a.kv_len[b]);
  if (len < 0) len = 0;
  const int nt = (int)cdiv(len, AF_KT);

  // Q fragments: query q0 + fr, head-dim slice [32 ks + 8 g, +8)
  bf16x8 qf[2];
  {
    const int64_t q = min(q0 + fr, a.Lq - 1);
    const bf16* Qp = reinterpret_cast<const bf16*>(a.q) + b * a.q_sb + h * a.q_sh + q * a.q_sl;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(Qp + ks * 32 + g * 8);
  }

  // K transfer of this lane: 1 KiB block `wid` of a tile = rows 8 wid .. 8 wid + 7
  const int k_row = wid * 8 + (lane >> 3);
  const bf16* k_src = Kb + ((lane & 7) ^ kswz(k_row)) * 8;
  // V of this lane: keys 2 kp, 2 kp + 1, head dims 4 dq .. 4 dq + 3; the two half-waves
  // take head-dim quads two apart (V^T rows 8 apart).
  const int half = lane >> 5, kp = lane & 31;
  const int dq = (wid & 1) + 4 * (wid >> 1) + 2 * half;
  const bf16* v_src = Vb + dq * 4;

  auto k_stage = [&](int j) { return smem + j * AF_KTILE; };
  auto v_stage = [&](int j) { return smem + AF_CH * AF_KTILE + j * AF_VTILE; };

  // fragment-read offsets inside a stage (constant over tiles)
  int k_off[4][2], v_off[2][4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int r = key_of(st, fr);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) k_off[st][ks] = r * 128 + (((ks * 4 + g) ^ kswz(r)) << 4);
  }
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 4; ++t) v_off[c][t] = (16 * t + fr) * AF_VP + (4 * c + g) * 16;

  float m_run = -INFINITY;
  f32x4 o_acc[4], l_acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 4; ++t) o_acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  bf16x8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = (bf16)1.0f;
  const float sl = a.scale_log2;

  for (int kc = 0; kc < nt; kc += AF_CH) {
    const int nc = min(AF_CH, nt - kc);
    if (kc > 0) __syncthreads();  // every wave is done with the previous chunk's stages
    // ---- issue every load of the chunk
    uint2 va[AF_CH], vb[AF_CH];
#pragma unroll
    for (int j = 0; j < AF_CH; ++j) {
      if (j < nc) {
        const int64_t k0 = (int64_t)(kc + j) * AF_KT;
        const int64_t kr = min(k0 + k_row, len - 1);
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(k_src + kr * a.k_sl),
                                         static_cast<void*>(k_stage(j) + wid * 1024), 16, 0, 0);
        const int64_t ka = min(k0 + 2 * kp, len - 1), kb = min(k0 + 2 * kp + 1, len - 1);
        va[j] = *reinterpret_cast<const uint2*>(v_src + ka * a.v_sl);
        vb[j] = *reinterpret_cast<const uint2*>(v_src + kb * a.v_sl);
      }
    }
    // ---- V^T: dword (V[2kp][4dq+e], V[2kp+1][4dq+e]) into row 4dq+e, column kp
#pragma unroll
    for (int j = 0; j < AF_CH; ++j) {
      if (j < nc) {
        unsigned char* base = v_stage(j) + (4 * dq) * AF_VP + kp * 4;
        const uint32_t a0 = va[j].x, a1 = va[j].y, b0 = vb[j].x, b1 = vb[j].y;
        *reinterpret_cast<uint32_t*>(base + 0 * AF_VP) = (a0 & 0xffffu) | (b0 << 16);
        *reinterpret_cast<uint32_t*>(base + 1 * AF_VP) = (a0 >> 16) | (b0 & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(base + 2 * AF_VP) = (a1 & 0xffffu) | (b1 << 16);
        *reinterpret_cast<uint32_t*>(base + 3 * AF_VP) = (a1 >> 16) | (b1 & 0xffff0000u);
      }
    }
    __syncthreads();  // K transfers landed and V^T written, for every wave

    for (int j = 0; j < nc; ++j) {
      const int kt = kc + j;
      const unsigned char* ks_ = k_stage(j);
      const unsigned char* vs_ = v_stage(j);
      f32x4 s[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x8 k0f = *reinterpret_cast<const bf16x8*>(ks_ + k_off[st][0]);
        const bf16x8 k1f = *reinterpret_cast<const bf16x8*>(ks_ + k_off[st][1]);
        f32x4 acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0f, qf[0], acc, 0, 0, 0);
        s[st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1f, qf[1], acc, 0, 0, 0);
      }
      const int64_t rem64 = len - (int64_t)kt * AF_KT;
      if (rem64 < AF_KT) {  // last, partial tile: mask keys past the sample's length
        const int rem = (int)rem64;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (32 * (st >> 1) + 8 * g + 4 * (st & 1) + i >= rem) s[st][i] = -INFINITY;
      }
      float mx = s[0][0];
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[st][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_tile = mx * sl;  // finite: every tile holds at least one valid key
      if (kt == 0) {
        m_run = m_tile;
      } else if (__any(m_tile > m_run + AF_RESCALE)) {  // wave-uniform: rare after the first tile
        const float m_new = fmaxf(m_run, m_tile);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_acc *= alpha;
#pragma unroll
        for (int t = 0; t < 4; ++t) o_acc[t] *= alpha;
      }
      bf16x8 pf[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[c][i] = (bf16)__builtin_amdgcn_exp2f(fmaf(s[2 * c][i], sl, -m_run));  // -inf -> 0
          pf[c][4 + i] = (bf16)__builtin_amdgcn_exp2f(fmaf(s[2 * c + 1][i], sl, -m_run));
        }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        l_acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[c], l_acc, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vs_ + v_off[c][t]);
          o_acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[c], o_acc[t], 0, 0, 0);
        }
      }
    }
  }

  const float l = l_acc[0];
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const int64_t q = q0 + fr;
  if (q < a.Lq) {
    bf16* O = reinterpret_cast<bf16*>(a.out) + b * a.o_sb + h * a.o_sh + q * a.o_sl;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      bf16x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (bf16)(o_acc[t][i] * inv);
      *reinterpret_cast<bf16x4*>(O + 16 * t + 4 * g) = v;
    }
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int try_attention_fast(const AttnArgs& a, int dtype, hipStream_t stream) {
  if (dtype != DT_BF16 || a.Dh != 64 || a.key_mask || a.block_mask) return 0;
  if (!(a.scale_log2 > 0.0f) || !(a.scale_log2 < INFINITY)) return 0;
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || ((uintptr_t)a.out & 7)) return 0;
  for (int64_t s : {a.q_sb, a.q_sh, a.q_sl, a.k_sb, a.k_sh, a.k_sl, a.v_sb, a.v_sh, a.v_sl})
    if (s % 8) return 0;
  for (int64_t s : {a.o_sb, a.o_sh, a.o_sl})
    if (s % 4) return 0;
  const int64_t nbh = a.B * a.H, nqb = cdiv(a.Lq, AF_QB);
  if (nbh > 65535 || nqb * nbh > 0x7fffffffLL) return 0;
  hipLaunchKernelGGL(attention_fast_kernel, dim3((unsigned)nqb, (unsigned)nbh), dim3(AF_THREADS), 0, stream, a);
  CORTEX_CHECK_LAUNCH("attention_fast_kernel");
  return 1;
}

}  // namespace cortex
