// Attention fast path for gfx950: bf16 operands, head dim 64, keys bounded by a
// per-sample length (dense self-attention, CSR cross-attention, broadcast queries)
// and optionally by a (block_l, block_e) tile mask with block_l % 16 == 0 and
// block_e % 64 == 0.  Every attention of the Cortex forward runs here; per-key
// padding masks, other tile shapes, fp32 and other head dims use the general kernel.
//
// Workgroup: 8 wavefronts x 16 or 32 queries of one (sample, head).  Keys are taken in
// chunks of up to 4 tiles of 64: every load of a chunk is issued at once (one
// memory round trip per chunk, not per tile), and each tile is multiplied as soon
// as its own loads have landed, while the later tiles' loads are still in flight.
// Two workgroups share a CU (64 KiB LDS each).
//
//   scores  S^T = K Q^T    (A = K rows from LDS, B = Q held in registers): a lane
//           holds 4 keys x 1 query per 16x16 sub-tile, so the softmax statistics of
//           a query are lane-local apart from two xor-shuffles (lane groups);
//   output  O^T += V^T P^T (A = V^T read transposed from LDS, B = P^T straight from the score
//           accumulators, rounded to bf16);
//   sums    l += 1 P^T     (an all-ones A operand: the key-sum of exactly the bf16
//           probabilities used in O, on the matrix core instead of the VALU).
//
// Key order.  Score sub-tile st, row r holds key 32(st/2) + 8(r/4) + 4(st%2) + r%4,
// so a lane of group g ends up with the 8 CONSECUTIVE keys 32c + 8g .. +7 for
// key step c: its V^T fragment is the 8 key rows 32c + 8g .. +7 at 4 head dims each.
//
// Staging.  K and V both go global -> LDS by direct transfers (buffer_load_dwordx4
// ... lds), row-major, 128 B a key row, the 16-byte chunk c of row r stored at c ^ f(r)
// (f = kswz for K, vswz for V) so that the rows one fragment read touches fall into
// distinct banks.  The V^T fragment comes out of the row-major V tile by two LDS
// transpose reads (ds_read_b64_tr_b16), each 4 key rows x 4 head dims of a 16-lane
// group.  No load of the tile loop has a register destination, so every wait on the
// transfers is an explicit vmcnt that counts tiles, and each tile is multiplied as
// soon as its own K and V have landed.
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
constexpr int AF_KTILE = AF_KT * 128;            // bytes of one K tile (64 keys x 64 bf16)
constexpr int AF_VTILE = AF_KT * 128;            // bytes of one V tile (64 keys x 64 bf16, row-major)
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

// s_waitcnt vmcnt(n) for the n of an unrolled tile index (lgkmcnt, expcnt untouched)
__device__ __forceinline__ void af_wait_vm(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0 | 0x70 | 0xF00); break;
    case 2: __builtin_amdgcn_s_waitcnt(2 | 0x70 | 0xF00); break;
    case 4: __builtin_amdgcn_s_waitcnt(4 | 0x70 | 0xF00); break;
    default: __builtin_amdgcn_s_waitcnt(6 | 0x70 | 0xF00); break;
  }
}

// V-tile chunk swizzle (16-byte chunks of a 128-byte key row): XOR with 2 h(r), h taking bits
// 1 and 3 of the row, so the 8 rows that a half-wavefront's transpose reads touch (rows
// 8 g + 0..3 of two lane groups, 32 bytes each) land on 8 distinct 32-byte bank ranges.
__device__ __forceinline__ int vswz(int r) { return (((r >> 1) & 1) | (((r >> 3) & 1) << 1)) << 1; }

// LDS transpose read (gfx950 ds_read_b64_tr_b16): in each group of 16 lanes, lane i gets
// element (i % 4) of the 4 elements at the address of lane 4 p + i / 4, for p = 0..3.
__device__ __forceinline__ uint2 lds_read_tr16(const unsigned char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Block-mask view of one sample: tile (qi, kj) is allowed iff m[qi * n_kt + kj] != 0;
// kj of a 64-key tile t is t / kpt (block_e = 64 kpt).
struct AfMask {
  const uint8_t* m;
  int64_t n_qt, n_kt, kpt;
  __device__ bool at(int64_t qi, int64_t kj) const {
    return qi >= 0 && qi < n_qt && kj < n_kt && m[qi * n_kt + kj] != 0;
  }
};

// 16-query groups per wavefront (QG): each K/V fragment read feeds QG MFMAs.  MASK: a
// (block_l, block_e) tile mask; the workgroup visits only the 64-key tiles that one of
// its query tiles allows, and a wavefront multiplies only those its own queries allow.
template <int QG, bool MASK>
__global__ __launch_bounds__(AF_THREADS) __attribute__((amdgpu_waves_per_eu(QG == 1 ? 4 : 2)))
void attention_fast_kernel(AttnArgs a) {
  constexpr int AF_QB = 16 * QG * AF_WAVES;  // queries per workgroup
  __shared__ __attribute__((aligned(1024))) unsigned char smem[AF_LDS];  // K tiles, then V tiles
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;

  // Keep the query blocks of one (sample, head) on one XCD (shared K/V in its L2).
  const int nqb = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + nqb * blockIdx.y, total);
  const int64_t bh = id / nqb;
  const int qblk = id % nqb;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t q0 = (int64_t)qblk * AF_QB + wid * (16 * QG);

  int64_t len = a.Lk;
  const bf16* Kb;
  const bf16* Vb;
  if (a.kv_off) {
    // offsets come from the caller: clamp them to the Lk key rows of the view
    const int64_t r0 = min(max(a.kv_off[b], (int64_t)0), a.Lk);
    len = min(max(a.kv_off[b + 1], r0), a.Lk) - r0;
    Kb = reinterpret_cast<const bf16*>(a.k) + r0 * a.k_sl + h * a.k_sh;
    Vb = reinterpret_cast<const bf16*>(a.v) + r0 * a.v_sl + h * a.v_sh;
  } else {
    Kb = reinterpret_cast<const bf16*>(a.k) + b * a.k_sb + h * a.k_sh;
    Vb = reinterpret_cast<const bf16*>(a.v) + b * a.v_sb + h * a.v_sh;
  }
  if (a.kv_len) len = min(len, a.kv_len[b]);
  if (len < 0) len = 0;
  len = wave_uniform(len);  // one (sample, head) per workgroup: the branches on it stay scalar
  const int nt = (int)cdiv(len, AF_KT);

  // Q fragments: query q0 + 16 qg + fr, head-dim slice [32 ks + 8 g, +8)
  bf16x8 qf[QG][2];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    const int64_t q = min(q0 + 16 * qg + fr, a.Lq - 1);
    const bf16* Qp = reinterpret_cast<const bf16*>(a.q) + b * a.q_sb + h * a.q_sh + q * a.q_sl;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qf[qg][ks] = *reinterpret_cast<const bf16x8*>(Qp + ks * 32 + g * 8);
  }

  // K transfer of this lane: 1 KiB block `wid` of a tile = rows 8 wid .. 8 wid + 7,
  // through a buffer resource based at the (sample, head) start: the byte offsets
  // stay below 2^32 (checked at launch).  Buffer transfers, unlike the global form,
  // leave the compiler's load counting exact for the V register loads.
  const int k_row = wid * 8 + (lane >> 3);
  const int64_t k_col = ((lane & 7) ^ kswz(k_row)) * 8;
  const __amdgpu_buffer_rsrc_t k_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(Kb), (short)0, (int)0xffffffffu, 0x00020000);
  // V transfer of this lane: the same rows as K, row-major into the V stage with the vswz
  // chunk swizzle (lane i: row 8 wid + i / 8, stored chunk i % 8 = logical (i % 8) ^ vswz(row))
  const int64_t v_col = ((lane & 7) ^ vswz(k_row)) * 8;
  const __amdgpu_buffer_rsrc_t v_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(Vb), (short)0, (int)0xffffffffu, 0x00020000);

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
  // V^T fragment (K block c, head dims 16 t ..): lane (fr, g) holds keys 32 c + 8 g + 0..7 of head
  // dim 16 t + fr, from two transpose reads 4 rows apart: each lane addresses row
  // 32 c + 8 g + fr / 4, head dims 16 t + 4 (fr % 4) .. +3 (vswz does not change over +4 rows)
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = 32 * c + 8 * g + (fr >> 2), d = 16 * t + 4 * (fr & 3);
      v_off[c][t] = r * 128 + (((d >> 3) ^ vswz(r)) << 4) + ((d >> 2) & 1) * 8;
    }

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

  // ---- tile schedule: the dense case takes tiles in order; with a mask, the tiles one
  // of the workgroup's query tiles allows, found 64 at a time by a ballot (every wave
  // computes the same, wave-uniform schedule).
  AfMask mk{};
  int64_t qrow[QG];  // query tile of each 16-query group
  int64_t qa = 0, qb = -1;  // query tiles of the workgroup
  if (MASK) {
    mk = AfMask{a.block_mask + b * a.bm_sb, a.n_qt, a.n_kt, a.block_e / AF_KT};
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) qrow[qg] = (q0 + 16 * qg) / a.block_l;
    qa = (int64_t)qblk * AF_QB / a.block_l;
    qb = min((int64_t)qblk * AF_QB + AF_QB - 1, a.Lq - 1) / a.block_l;
  }
  auto wg_window = [&](int base) -> uint64_t {  // allowed tiles base .. base + 63
    const int t = base + lane;
    bool ok = false;
    if (t < nt) {
      const int64_t kj = t / mk.kpt;
      for (int64_t qi = qa; qi <= qb && !ok; ++qi) ok = mk.at(qi, kj);
    }
    return __ballot(ok);
  };
  int wbase = 0;
  uint64_t pend = MASK ? wg_window(0) : 0;

  const uint32_t k_lane = (uint32_t)(((int64_t)k_row * a.k_sl + k_col) * 2);
  const uint32_t v_lane = (uint32_t)(((int64_t)k_row * a.v_sl + v_col) * 2);
  // ---- the loads of tile t (keys clamped to the sample) into stage j: the K and V transfers,
  // both direct to LDS, so no load in flight has a register destination and the waits below
  // count exactly (with the V rows in registers, the compiler waited for every load in flight
  // before their use, emptying the ring).  With 32 queries per wavefront a whole tile takes a
  // uniform tile offset plus the lane's constant offsets; the sample's last, partial tile
  // clamps its rows.
  auto issue_tile = [&](int t, int j) {
    const int64_t k0 = (int64_t)t * AF_KT;
    uint32_t koff, voff;
    if (QG == 2 && k0 + AF_KT <= len) {
      koff = (uint32_t)(k0 * a.k_sl * 2) + k_lane;
      voff = (uint32_t)(k0 * a.v_sl * 2) + v_lane;
    } else {
      const int64_t kr = min(k0 + k_row, len - 1);
      koff = (uint32_t)((kr * a.k_sl + k_col) * 2);
      voff = (uint32_t)((kr * a.v_sl + v_col) * 2);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        k_rsrc, (__attribute__((address_space(3))) void*)(k_stage(j) + wid * 1024), 16, (int)koff, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        v_rsrc, (__attribute__((address_space(3))) void*)(v_stage(j) + wid * 1024), 16, (int)voff, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order tile by tile (vmcnt below)
  };
  // ---- scores S^T = K Q^T of the key tile in stage j (16-query groups with okq set)
  typedef f32x4 Scores[QG][4];
  auto scores = [&](int j, const bool (&okq)[QG], Scores& s) {
    const unsigned char* ks_ = k_stage(j);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bf16x8 k0f = *reinterpret_cast<const bf16x8*>(ks_ + k_off[st][0]);
      const bf16x8 k1f = *reinterpret_cast<const bf16x8*>(ks_ + k_off[st][1]);
#pragma unroll
      for (int qg = 0; qg < QG; ++qg) {
        f32x4 acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        if (!okq[qg]) continue;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0f, qf[qg][0], acc, 0, 0, 0);
        s[qg][st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1f, qf[qg][1], acc, 0, 0, 0);
      }
    }
  };
  // ---- online softmax of the scores of key tile kt, then P V with its V^T in stage j
  auto softmax_pv = [&](int kt, int j, const bool (&okq)[QG], Scores& s) {
    const unsigned char* vs_ = v_stage(j);
    const int64_t rem64 = len - (int64_t)kt * AF_KT;
    if (rem64 < AF_KT) {  // last, partial tile: mask keys past the sample's length
      const int rem = (int)rem64;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (32 * (st >> 1) + 8 * g + 4 * (st & 1) + i >= rem) {
#pragma unroll
            for (int qg = 0; qg < QG; ++qg) s[qg][st][i] = -INFINITY;
          }
    }
    bf16x8 pf[QG][2];
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) {
      if (!okq[qg]) continue;
      // Lane-local max first: the reference max only has to move (and the lane groups
      // only have to agree on a new one) when some score exceeds it by AF_RESCALE.
      float mx = s[qg][0][0];
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[qg][st][i]);
      // wave-uniform, rare after the group's first tile (m_run = -inf always enters)
      if (__any(mx * sl > m_run[qg] + AF_RESCALE)) {
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_tile = mx * sl;  // finite: every tile holds at least one valid key
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
          pf[qg][c][i] = (bf16)__builtin_amdgcn_exp2f(fmaf(s[qg][2 * c][i], sl, -m_run[qg]));  // -inf -> 0
          pf[qg][c][4 + i] = (bf16)__builtin_amdgcn_exp2f(fmaf(s[qg][2 * c + 1][i], sl, -m_run[qg]));
        }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int qg = 0; qg < QG; ++qg)
        if (okq[qg]) l_acc[qg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[qg][c], l_acc[qg], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint2 v0 = lds_read_tr16(vs_ + v_off[c][t]), v1 = lds_read_tr16(vs_ + v_off[c][t] + 4 * 128);
        const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(v0.x, v0.y, v1.x, v1.y));
#pragma unroll
        for (int qg = 0; qg < QG; ++qg)
          if (okq[qg]) o_acc[qg][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[qg][c], o_acc[qg][t], 0, 0, 0);
      }
    }
  };
  // the tile-mask path: scores, softmax and P V of tile kt in stage j, one after the other
  auto do_tile = [&](int kt, int j) {
    bool okq[QG];  // this 16-query group multiplies tile kt
    bool any = false;
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) {
      okq[qg] = mk.at(qrow[qg], kt / mk.kpt);
      any = any || okq[qg];
    }
    if (!any) return;
    Scores s;
    scores(j, okq, s);
    softmax_pv(kt, j, okq, s);
  };

  if constexpr (!MASK) {
    // Dense keys: the stages form a ring, and the tiles are software-pipelined.  Tiles 0..3
    // are issued up front.  Iteration kt makes tile kt + 1 visible (its transfers awaited, barrier),
    // issues its score MFMAs, and only then runs the softmax and P V of tile kt, whose scores
    // the previous iteration produced: the matrix core works on tile kt + 1 while the VALU
    // evaluates tile kt's exponentials.  After that barrier every wavefront is done with tile
    // kt - 1, so its stage is refilled with tile kt + 3 (clamped past the end: issued, never
    // read).  Each tile is 2 transfers; the waits name the tiles issued after the awaited one.
    bool all[QG];
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) all[qg] = true;
    Scores sc[2];
    if (nt > 0) {  // (no keys: nothing is loaded, the rows give 0)
#pragma unroll
      for (int t = 0; t < AF_CH; ++t) issue_tile(min(t, nt - 1), t);
      af_wait_vm(6);
      __builtin_amdgcn_s_barrier();
      scores(0, all, sc[0]);
    }
    for (int kt0 = 0; kt0 < nt; kt0 += AF_CH) {
#pragma unroll
      for (int t = 0; t < AF_CH; ++t) {
        const int kt = kt0 + t;
        if (kt >= nt) break;
        const int tn = (t + 1) & 3;  // stage of tile kt + 1
        if (kt + 1 < nt) {
          af_wait_vm(kt == 0 ? 4 : 2);
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): tile kt-1's reads done
          __builtin_amdgcn_s_barrier();        // tile kt+1 visible; stage of tile kt-1 free
          if (kt >= 1) issue_tile(min(kt + 3, nt - 1), (t + 3) & 3);
          scores(tn, all, sc[(t + 1) & 1]);
        }
        softmax_pv(kt, t, all, sc[t & 1]);
      }
    }
  } else {
    // Tile mask: the workgroup's allowed tiles come from ballot windows, taken in chunks of
    // AF_CH tiles whose loads are all issued at once.
    for (bool first = true;; first = false) {
      int tl[AF_CH];
      int nc = 0;
#pragma unroll
      for (int j = 0; j < AF_CH; ++j) {
        while (pend == 0 && wbase + 64 < nt) {
          wbase += 64;
          pend = wg_window(wbase);
        }
        if (pend != 0) {
          tl[j] = wbase + __builtin_ctzll(pend);
          pend &= pend - 1;
          nc = j + 1;
        } else {
          tl[j] = j > 0 ? tl[j - 1] : 0;  // loaded, never used
        }
      }
      if (nc <= 0) break;
      if (!first) __syncthreads();  // every wave is done with the previous chunk's stages
      // Stages past the chunk's last tile are filled too (clamped keys) and never read:
      // unconditional issue keeps the load counter exact, so each tile below waits for its
      // own loads only (vmcnt(3 (AF_CH-1-j)): tile j's K transfer and V registers are in).
#pragma unroll
      for (int j = 0; j < AF_CH; ++j) issue_tile(tl[j], j);
#pragma unroll
      for (int j = 0; j < AF_CH; ++j) {
        if (j >= nc) break;
        af_wait_vm(2 * (AF_CH - 1 - j));
        __builtin_amdgcn_s_barrier();        // tile j's K and V transfers visible to all
        do_tile(tl[j], j);
      }
    }
  }
  af_wait_vm(0);  // the last chunk's unused stages: no transfer into LDS outlives the workgroup
  // the last element of the output view, in bytes from its base
  const int64_t o_bytes = ((a.B - 1) * a.o_sb + (a.H - 1) * a.o_sh + (a.Lq - 1) * a.o_sl + a.Dh) * 2;
  const WtOut store(a.out, o_bytes, wt_one_wave());

#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    const float l = l_acc[qg][0];
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int64_t q = q0 + 16 * qg + fr;
    if (q < a.Lq) {
      bf16* O = reinterpret_cast<bf16*>(a.out) + b * a.o_sb + h * a.o_sh + q * a.o_sl;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (bf16)(o_acc[qg][t][i] * inv);
        store(reinterpret_cast<bf16x4*>(O + 16 * t + 4 * g), v);
      }
    }
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int try_attention_fast(const AttnArgs& a, int dtype, hipStream_t stream) {
  if (dtype != DT_BF16 || a.Dh != 64 || a.key_mask) return 0;
  // a tile mask must give each 16-query group and each 64-key tile one mask entry
  const bool mask = a.block_mask != nullptr;
  if (mask && (a.block_l % 16 != 0 || a.block_e % AF_KT != 0 || a.n_qt <= 0 || a.n_kt <= 0)) return 0;
  if (!(a.scale_log2 > 0.0f) || !(a.scale_log2 < INFINITY)) return 0;
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || ((uintptr_t)a.out & 7)) return 0;
  for (int64_t s : {a.q_sb, a.q_sh, a.q_sl, a.k_sb, a.k_sh, a.k_sl, a.v_sb, a.v_sh, a.v_sl})
    if (s % 8) return 0;
  for (int64_t s : {a.o_sb, a.o_sh, a.o_sl})
    if (s % 4) return 0;
  const int64_t nbh = a.B * a.H;
  // 32 queries per wavefront (K/V fragments read once per two MFMAs) while that still
  // gives every CU a workgroup; 16 otherwise
  const int qg = cdiv(a.Lq, 16 * 2 * AF_WAVES) * nbh >= 256 ? 2 : 1;
  const int64_t nqb = cdiv(a.Lq, 16 * qg * AF_WAVES);
  if (nbh > 65535 || nqb * nbh > 0x7fffffffLL) return 0;
  // K and V byte offsets from a (sample, head) start are 32-bit buffer offsets
  if (a.Lk > 0 && ((a.Lk - 1) * a.k_sl * 2 + 128 > 0xffffffffLL || (a.Lk - 1) * a.v_sl * 2 + 128 > 0xffffffffLL))
    return 0;
  const dim3 grid((unsigned)nqb, (unsigned)nbh);
  if (qg == 2 && mask)
    hipLaunchKernelGGL((attention_fast_kernel<2, true>), grid, dim3(AF_THREADS), 0, stream, a);
  else if (qg == 2)
    hipLaunchKernelGGL((attention_fast_kernel<2, false>), grid, dim3(AF_THREADS), 0, stream, a);
  else if (mask)
    hipLaunchKernelGGL((attention_fast_kernel<1, true>), grid, dim3(AF_THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL((attention_fast_kernel<1, false>), grid, dim3(AF_THREADS), 0, stream, a);
  CORTEX_CHECK_LAUNCH("attention_fast_kernel");
  return 1;
}

}  // namespace cortex
