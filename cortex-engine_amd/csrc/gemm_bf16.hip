// bf16 x bf16 (and int8 x int8) GEMM for gfx950 with direct-to-LDS operand streaming
// and a register epilogue:
//
//   C[m, n] = epi( sum_k A[m, k] * W[n, k] ),  A (M, K) bf16 rows, W (N, K) bf16 rows
//   epi: * w_scale[n] (+ bias[n]) (-> erf-GELU) -> bf16 | fp32, or (+ fp32 residual) -> fp32
//
// W is the bf16 execution image of a QuantizedLinear's int8 weight (exact) with the
// per-channel scale applied in the epilogue, or a float weight rounded to bf16.
//
// The int8 form (TIN = int8_t: the opt-in W8A8 mode) takes int8 activation rows
// x = round(x_f / a_scale) and the int8 weight itself, accumulates exactly in int32 on
// v_mfma_i32_16x16x64_i8 and applies a_scale * w_scale[n] in the epilogue; its outputs
// are fp32 (with the residual) or int8 at the next linear's activation scale.  Both
// MFMAs read 16 bytes per lane per operand, so the LDS ring, swizzles and transfers are
// byte-for-byte the same; a 128-byte LDS row holds 64 bf16 or 128 int8 of K.
//
// Operands travel global -> LDS with global_load_lds_dwordx4 (1 KiB per wavefront
// instruction, no VGPRs held while in flight) through a STAGES-deep ring; a step
// waits only for its own transfers (vmcnt) plus a raw s_barrier.
//
// LDS rows hold 128 bytes of K; the 16-byte chunk c of row r is stored at
// c ^ sw(r), with sw chosen so that the 16 rows read by one MFMA fragment cover all
// 16 four-bank groups.
//
// The MFMA computes C^T tiles (A operand = W rows, B operand = A rows) with the W
// rows of two adjacent tiles interleaved, so a lane ends up with 8 CONSECUTIVE
// output columns of one row: the epilogue reads scale, bias and residual as float4
// pairs and writes 16- or 32-byte vectors straight from the accumulators, without
// an LDS round trip or a workgroup barrier.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "common.h"
#include "gemm.h"

namespace cortex {

namespace {

template <int n>
__device__ __forceinline__ void wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | 0x70 | 0xF00 | ((n >> 4) << 14));
}

// pair d (values 2d, 2d + 1) of eight bf16 values, for the two-term dot products
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x2_t pair_of(const bf16x8& v, int d) {
  switch (d) {
    case 0: return __builtin_shufflevector(v, v, 0, 1);
    case 1: return __builtin_shufflevector(v, v, 2, 3);
    case 2: return __builtin_shufflevector(v, v, 4, 5);
    default: return __builtin_shufflevector(v, v, 6, 7);
  }
}

// Direct-to-LDS transfer from a uniform base plus a 32-bit lane offset (global_load_lds in its
// scalar-base form: one VGPR per transfer instead of a 64-bit address) into the LDS address m0
// (wave-uniform: lane i writes m0 + SIZE * i), SIZE 16 (dwordx4) or 4 (dword).  The caller's
// vmcnt waits order the reads.
template <int SIZE>
__device__ __forceinline__ void lds_dma_m0(const void* base, uint32_t voff, uint32_t m0) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  const uint32_t m = __builtin_amdgcn_readfirstlane(m0);
  if constexpr (SIZE == 16)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb), "s"(m)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sb), "s"(m)
                 : "memory", "m0");
}

// KS > 1 splits K over KS groups of WM x WN wavefronts, each streaming its own part of
// K through its own LDS ring; the partial tiles are summed through LDS before the
// epilogue.  This doubles the wavefronts per CU for narrow outputs (N = 512) without
// shrinking the wavefront tiles.
template <int BM_, int BN_, int STAGES_, int WM_, int WN_, int KS_ = 1>
struct BTile {
  static constexpr int BM = BM_, BN = BN_, BK = 64, STAGES = STAGES_, WM = WM_, WN = WN_, KS = KS_;
  static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES * KS;  // WAVES: per K group
  static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16x16 tiles per wavefront
  static constexpr int A_STAGE = BM * 128, W_STAGE = BN * 128;  // bytes (rows of 64 bf16)
  static constexpr int A_BLOCKS = A_STAGE / 1024 / WAVES, W_BLOCKS = W_STAGE / 1024 / WAVES;
  static constexpr int PER = A_BLOCKS + W_BLOCKS;              // transfers per wavefront per step
  static constexpr int RING = STAGES * (A_STAGE + W_STAGE);     // bytes per K group
  static constexpr int RED = (KS > 1) ? WAVES * TM * TN * 4 * 64 * 4 : 0;  // partial tile exchange
  static constexpr int LDS = (KS * RING > RED) ? KS * RING : RED;
  static_assert(KS == 1 || KS == 2, "K split");
  static_assert(A_STAGE % (1024 * WAVES) == 0 && W_STAGE % (1024 * WAVES) == 0, "transfer split");
  static_assert(TM >= 1 && TN >= 2 && TN % 2 == 0 && STAGES >= 2, "shape");
  static_assert(PER * (STAGES - 1) < 64, "vmcnt range");
};

// 16-byte chunk swizzles of the 128-byte LDS rows.  A fragments read 16 consecutive
// rows; W fragments read rows 8q + 4jj + i (q, i in 0..3) -- see the column order
// below.  Each swizzle puts its fragment's 16 rows into the 16 distinct (row parity,
// chunk) four-bank groups.
__device__ __forceinline__ int swz_a(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swz_w(int r) { return ((r >> 1) & 1) | ((r >> 2) & 6); }

// Column order.  W fragment row rho (0..15) of tile 2p + jj of a wavefront holds
// output column 32 p + 8 (rho / 4) + 4 jj + rho % 4, so that the accumulators of
// tiles 2p and 2p+1 give lane group g4 the 8 consecutive columns 32 p + 8 g4 .. +7.
__device__ __forceinline__ int wrow_of(int p, int jj, int rho) { return 32 * p + 8 * (rho >> 2) + 4 * jj + (rho & 3); }

// int8 weight rows with bf16 activations (TW = int8_t, TIN = bf16: the QuantizedLinear int8
// weight itself): the int8 rows travel global -> LDS by the same direct-to-LDS transfers as
// bf16 rows, 64 bytes of K per row and step (half the bytes), and each lane widens its 8-byte
// fragment exactly to bf16 (every int8 value is a bf16 value; one byte convert per value and
// one pack per pair) right before the MFMAs that use it.  The 16-byte chunk c of LDS row r
// holds logical chunk c ^ swz8(r): the 16 rows of one fragment read then fall on distinct
// four-bank groups in both output orders (natural rows 0..15, interleaved rows of wrow_of).
__device__ __forceinline__ int swz8(int r) { return ((r >> 3) ^ (r >> 2)) & 3; }

template <class TL, int ACT, bool RES, class TOUT, class TIN = bf16, class TW = TIN, bool RS = false>
__global__ __launch_bounds__(TL::THREADS) void gemm_bf16_kernel(GemmArgs g) {
  constexpr int BM = TL::BM, BN = TL::BN, TM = TL::TM, TN = TL::TN, S = TL::STAGES;
  constexpr int AB = TL::A_BLOCKS, WB = TL::W_BLOCKS, PER = TL::PER;
  // bf16 / int8 output: interleaved W rows, 8 consecutive columns per lane;
  // fp32 output: natural order, 4 consecutive columns (16 bytes) per lane and tile.
  constexpr bool IL = sizeof(TOUT) <= 2;
  using OP = Operand<TIN>;
  typedef typename OP::frag frag;
  constexpr int EPC = OP::EPC, BK = 8 * EPC;  // K elements per 16-byte chunk and per 128-byte row
  // int8 weight rows through LDS, widened at the fragment read (see swz8): 64-byte rows, so a
  // stage holds BN * 64 bytes of W and a wavefront transfers W8B 1 KiB blocks per step
  constexpr bool WI8 = sizeof(TW) == 1 && sizeof(TIN) == 2;
  constexpr int W_STAGE = WI8 ? BN * 64 : TL::W_STAGE;
  constexpr int W8B = WI8 ? W_STAGE / 1024 / TL::WAVES : 1;
  static_assert(!WI8 || W_STAGE % (1024 * TL::WAVES) == 0, "int8 weight transfer split");
  // RS: each lane sums the squares of the A values its fragments hold (row wrow + 16 t + fr,
  // eight of every 32 K per sub-step); the four lanes of a row complete the sum at the end
  static_assert(!RS || (sizeof(TIN) == 2 && sizeof(TW) == 2 && !RES), "row scale: bf16 operands");
  constexpr int WOPS = WI8 ? W8B : WB;  // vector-memory operations per step for W
  constexpr int STEP_OPS = AB + WOPS;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[TL::LDS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int kg = (tid >> 6) / TL::WAVES, wid = (tid >> 6) % TL::WAVES;  // K group, wave within it
  const int wm = wid / TL::WN, wn = wid % TL::WN;
  const int nbx = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + nbx * blockIdx.y, total);  // contiguous row tiles per XCD
  const int m0 = (id / nbx) * BM, n0 = (id % nbx) * BN;
  unsigned char* const ring = smem + kg * TL::RING;
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  // K split across workgroups (split_k_partials): slice z of K into output slab z
  const int kz = blockIdx.z;
  const TIN* __restrict__ A = reinterpret_cast<const TIN*>(g.x) + (int64_t)kz * K;
  const TW* __restrict__ W = reinterpret_cast<const TW*>(g.w) + (int64_t)kz * K;

  // Global source of each of this lane's transfers (K offset added per step).  Lane i
  // of a transfer writes LDS bytes [16 i, 16 i + 16) of its 1 KiB block: row i / 8,
  // stored chunk i % 8, which holds logical chunk (i % 8) ^ swizzle(row).
  // RS: 32-bit byte offsets from the uniform operand bases instead of 64-bit pointers (the
  // transfers take the scalar-base form, and the kernel stays within its registers; the host
  // keeps both operands below 4 GiB)
  constexpr bool O32 = RS;
  const TIN* a_src[O32 ? 1 : AB];
  uint32_t a_vo[O32 ? AB : 1];
#pragma unroll
  for (int i = 0; i < AB; ++i) {
    const int r = (wid * AB + i) * 8 + (lane >> 3);
    const int64_t e = (int64_t)min(m0 + r, M - 1) * g.ld_x + ((lane & 7) ^ swz_a(r)) * EPC;
    if constexpr (O32) a_vo[i] = (uint32_t)(e * (int64_t)sizeof(TIN));
    else a_src[i] = A + e;
  }
  const TW* w_src[O32 ? 1 : (WI8 ? W8B : WB)];
  uint32_t w_vo[O32 ? WB : 1];
  if constexpr (WI8) {
    // lane i of block q writes LDS bytes [16 i, 16 i + 16): row 16 q + i / 4, stored chunk i % 4
#pragma unroll
    for (int i = 0; i < W8B; ++i) {
      const int r = (wid * W8B + i) * 16 + (lane >> 2);
      w_src[i] = W + (int64_t)min(n0 + r, N - 1) * g.ld_w + (((lane & 3) ^ swz8(r)) * 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < WB; ++i) {
      const int r = (wid * WB + i) * 8 + (lane >> 3);
      const int64_t e = (int64_t)min(n0 + r, N - 1) * g.ld_w + ((lane & 7) ^ (IL ? swz_w(r) : swz_a(r))) * EPC;
      if constexpr (O32) w_vo[i] = (uint32_t)(e * (int64_t)sizeof(TW));
      else w_src[i] = W + e;
    }
  }
  auto a_stage = [&](int s) { return ring + s * TL::A_STAGE; };
  auto w_stage = [&](int s) { return ring + S * TL::A_STAGE + s * W_STAGE; };
  const int nk = K / BK / TL::KS;  // K steps of this group
  const int kbase = kg * nk * BK;
  auto issue = [&](int kt) {
    const int s = kt % S, k0 = kbase + kt * BK;
    if constexpr (WI8) {
#pragma unroll
      for (int i = 0; i < W8B; ++i)
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(w_src[i] + k0),
                                         static_cast<void*>(w_stage(s) + (wid * W8B + i) * 1024), 16, 0, 0);
    }
    if constexpr (O32) {
      // LDS destinations as wave-uniform 32-bit addresses (no per-lane generic pointers)
      const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ring);
      const int wu = __builtin_amdgcn_readfirstlane(wid);
#pragma unroll
      for (int i = 0; i < AB; ++i) lds_dma_m0<16>(A + k0, a_vo[i], ring0 + s * TL::A_STAGE + (wu * AB + i) * 1024);
#pragma unroll
      for (int i = 0; i < WB; ++i)
        lds_dma_m0<16>(W + k0, w_vo[i], ring0 + S * TL::A_STAGE + s * W_STAGE + (wu * WB + i) * 1024);
      return;
    }
#pragma unroll
    for (int i = 0; i < AB; ++i)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(a_src[i] + k0),
                                       static_cast<void*>(a_stage(s) + (wid * AB + i) * 1024), 16, 0, 0);
    if constexpr (!WI8) {
#pragma unroll
      for (int i = 0; i < WB; ++i)
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(w_src[i] + k0),
                                         static_cast<void*>(w_stage(s) + (wid * WB + i) * 1024), 16, 0, 0);
    }
  };

  typename OP::accum acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (typename OP::accum){0, 0, 0, 0};

  const int fr = lane & 15, g4 = lane >> 4;
  const int wrow = wm * (BM / TL::WM), wcol = wn * (BN / TL::WN);
  // fragment-read byte offsets inside a stage (row base) and the row swizzles
  int a_off[TM], w_off[TN], a_sw[TM], w_sw[TN];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int r = wrow + t * 16 + fr;
    a_off[t] = r * 128;
    a_sw[t] = swz_a(r);
  }
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int r = wcol + (IL ? wrow_of(t >> 1, t & 1, fr) : t * 16 + fr);
    w_off[t] = r * (WI8 ? 64 : 128);
    w_sw[t] = WI8 ? swz8(r) : IL ? swz_w(r) : swz_a(r);
  }
  // W fragments as read from LDS: bf16 fragments, or with int8 weights the raw 8 bytes, widened
  // in the MFMA loop right before their TM uses (double-buffered raw bytes take half the
  // registers of widened fragments)
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
  float ssq[RS ? TM : 1] = {};  // RS: this lane's sum of squares of each row fragment
  // Raised wave priority over each MFMA group, so a wavefront ready to multiply issues ahead of
  // its SIMD partner's fragment reads and transfers.  Measured per kernel: it pays for the
  // row-scaled form with the K split (config 2 at N = 512: 9.75 -> 9.29 us) and costs the
  // single-group tiles and the residual GEMMs 0.4-1 us, so only that form sets it.
  constexpr bool PRIO = RS && TL::KS > 1;
  auto mma = [&](const frag (&af)[TM], const wfrag (&wf)[TN]) {
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
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
        for (int j = 0; j < TN; ++j)
          acc[i][j] = OP::mma(wf[j], af[i], acc[i][j]);
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    if constexpr (RS) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const bf16x2_t xv = pair_of(af[i], d);
          ssq[i] = __builtin_amdgcn_fdot2_f32_bf16(xv, xv, ssq[i], false);
        }
    }
  };

  // The residual tile is fetched into registers before the main loop, so its latency
  // hides behind the MFMAs instead of stalling the epilogue.
  const float* res = reinterpret_cast<const float*>(g.res);
  const int res_rows = g.res_rows > 0 ? (int)g.res_rows : M;
  float4 rv[RES ? TM : 1][RES ? TN : 1];
  if constexpr (RES && !IL) {
    if (kg == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = min(m0 + wrow + i * 16 + fr, M - 1);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = min(n0 + wcol + 16 * j + 4 * g4, N - 4);
        rv[i][j] = *reinterpret_cast<const float4*>(res + (int64_t)(m % res_rows) * g.ld_res + n);
      }
    }
    }
  }

  // Every stage of the ring is in flight at once; a stage is refilled as soon as all
  // wavefronts hold its last fragments in registers.  Fragments are double-buffered
  // in registers, so the LDS reads of the next K sub-step overlap the MFMAs.
#pragma unroll
  for (int p = 0; p < S; ++p)
    if (p < nk) issue(p);
  // wait until this wave's transfers of step j landed, steps up to `last` being issued
  auto wait_step = [&](int j, int last) {
    const int ahead = min(nk - 1, last) - j;  // steps issued after j
    if constexpr (S >= 3) {
      if (ahead >= 2)
        wait_vm<2 * STEP_OPS>();
      else if (ahead == 1)
        wait_vm<STEP_OPS>();
      else
        wait_vm<0>();
    } else {
      if (ahead >= 1)
        wait_vm<STEP_OPS>();
      else
        wait_vm<0>();
    }
  };
  frag af0[TM], af1[TM];
  wfrag wf0[TN], wf1[TN];
  wait_step(0, S - 1);
  __builtin_amdgcn_s_barrier();
  read_frags(0, 0, af0, wf0);
  // One K step that hands over to the next: sub-step 1's fragments are read while sub-step 0
  // multiplies; after the barrier, the next step's sub-step 0 fragments (and the refill of
  // the freed stage) are issued before sub-step 1 multiplies.  The loop is peeled (steps
  // that refill, steps that do not, the last step) so that no branch joins in front of an
  // MFMA group: at a join the compiler waits for every LDS read in flight, including the ones
  // just issued, and the double-buffered fragments would no longer overlap the MFMAs.  Each
  // step starts with an explicit wait for the fragments read after the previous barrier, for
  // the same reason (the compiler cannot track them across the loop's back edge).
  auto step = [&](int kt, auto refill) {
    const int st = kt % S;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): sub-step 0's fragments
    read_frags(st, 1, af1, wf1);
    __builtin_amdgcn_sched_barrier(0);   // the reads go out first: the barrier below waits for them
    mma(af0, wf0);
    __builtin_amdgcn_sched_barrier(0);   // and every MFMA of sub-step 0 is issued before that wait
    wait_step(kt + 1, kt + S - 1);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage st done
    __builtin_amdgcn_s_barrier();        // all waves done with stage st; step kt+1 visible
    read_frags((kt + 1) % S, 0, af0, wf0);
    __builtin_amdgcn_sched_barrier(0);   // the next step's first reads go out before these MFMAs
    if constexpr (decltype(refill)::value) issue(kt + S);  // refill stage st
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

  if constexpr (TL::KS > 1) {
    // group 1 hands its partial tile to group 0 through LDS: one 16-byte access per accumulator
    // fragment, lane-contiguous (conflict free)
    typename OP::accum* red4 = reinterpret_cast<typename OP::accum*>(smem);
    float* red_ss = reinterpret_cast<float*>(smem + TL::RED);  // RS: the partial sums of squares
    static_assert(!RS || TL::RED + TL::WAVES * TM * 64 * 4 <= TL::LDS, "exchange area");
    __syncthreads();  // every ring read is done; the exchange area may overwrite the rings
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) red4[((wid * TM + i) * TN + j) * 64 + lane] = acc[i][j];
      if constexpr (RS) {
#pragma unroll
        for (int i = 0; i < TM; ++i) red_ss[(wid * TM + i) * 64 + lane] = ssq[i];
      }
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] += red4[((wid * TM + i) * TN + j) * 64 + lane];
    if constexpr (RS) {
#pragma unroll
      for (int i = 0; i < TM; ++i) ssq[i] += red_ss[(wid * TM + i) * 64 + lane];
    }
  }

  float rinv[RS ? TM : 1];
  if constexpr (RS) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float s1 = ssq[i];
      s1 += __shfl_xor(s1, 16, 64);
      s1 += __shfl_xor(s1, 32, 64);
      rinv[i] = 1.0f / sqrtf(s1 / (float)K + g.rms_eps);
    }
  }
  auto row_scaled = [&](float a, int i) {
    if constexpr (RS) return a * rinv[i];
    else return a;
  };

  // ---- epilogue from registers.  Row m0 + wrow + 16 i + fr; columns
  //   IL:  tiles 2p, 2p+1 -> n0 + wcol + 32 p + 8 g4 .. +7
  //   !IL: tile j         -> n0 + wcol + 16 j + 4 g4 .. +3
  const float* bias = reinterpret_cast<const float*>(g.bias);
  TOUT* out = reinterpret_cast<TOUT*>(g.out) + (int64_t)kz * M * g.ld_out;
  const WtOut store(out, (int64_t)M * g.ld_out * (int64_t)sizeof(TOUT), wt_one_wave());
  // the lane's first output row once; each further 16-row group adds a uniform step, kept
  // opaque so that the compiler does not fold it back into a 64-bit multiply per store
  const int64_t row_base = (int64_t)(m0 + wrow + fr) * g.ld_out;
  const int64_t step16 =
      (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(g.ld_out >> 28)) << 32) |
                (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(g.ld_out << 4)));
  constexpr int NV = IL ? 8 : 4;           // consecutive columns per lane and group
  constexpr int NG = IL ? TN / 2 : TN;     // column groups per lane
  // Every scale and bias load first, then one wait: a wait left to the compiler would
  // sit at each row's branch and also drain the previous row's stores.
  float sca[NG][NV], bia[NG][NV];
#pragma unroll
  for (int p = 0; p < NG; ++p) {
    const int n = min(n0 + wcol + (IL ? 32 * p + 8 * g4 : 16 * p + 4 * g4), N - NV);
#pragma unroll
    for (int h = 0; h < NV / 4; ++h) {
      float4 s4 = g.w_scale ? *reinterpret_cast<const float4*>(g.w_scale + n + 4 * h)
                            : make_float4(1.f, 1.f, 1.f, 1.f);
      if constexpr (sizeof(TIN) == 1) {  // int8 activations: x_f = a_scale * x
        s4.x *= g.a_scale; s4.y *= g.a_scale; s4.z *= g.a_scale; s4.w *= g.a_scale;
      }
      const float4 b4 = bias ? *reinterpret_cast<const float4*>(bias + n + 4 * h) : make_float4(0.f, 0.f, 0.f, 0.f);
      sca[p][4 * h] = s4.x; sca[p][4 * h + 1] = s4.y; sca[p][4 * h + 2] = s4.z; sca[p][4 * h + 3] = s4.w;
      bia[p][4 * h] = b4.x; bia[p][4 * h + 1] = b4.y; bia[p][4 * h + 2] = b4.z; bia[p][4 * h + 3] = b4.w;
    }
  }
  wait_vm<0>();
#pragma unroll
  for (int p = 0; p < NG; ++p) {
    const int n = n0 + wcol + (IL ? 32 * p + 8 * g4 : 16 * p + 4 * g4);
    if (n >= N) continue;  // N % 8 == 0: a lane's columns are all in or all out
    const float* sc = sca[p];
    const float* bi = bia[p];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wrow + i * 16 + fr;
      if (m >= M) continue;
      float v[NV];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (IL) {
          v[r] = row_scaled(acc[i][2 * p][r], i) * sc[r] + bi[r];
          v[4 + r] = row_scaled(acc[i][2 * p + 1][r], i) * sc[4 + r] + bi[4 + r];
        } else {
          v[r] = row_scaled(acc[i][p][r], i) * sc[r] + bi[r];
        }
      }
      if (ACT == ACT_GELU) {
#pragma unroll
        for (int e = 0; e < NV; ++e) v[e] = sizeof(TOUT) <= 2 ? gelu_erf_bf16out(v[e]) : gelu_erf(v[e]);
      }
      if constexpr (RES && !IL) {
        const float4 x = rv[i][p];
        v[0] += x.x; v[1] += x.y; v[2] += x.z; v[3] += x.w;
      }
      TOUT* op = out + (row_base + i * step16 + n);
      if constexpr (sizeof(TOUT) == 2) {
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (bf16)v[e];
        store(reinterpret_cast<bf16x8*>(op), o);
      } else if constexpr (sizeof(TOUT) == 1) {  // int8 at the next linear's activation scale
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int q0 = (int)fminf(fmaxf(rintf(v[e] * g.out_inv_scale), -127.0f), 127.0f);
          const int q1 = (int)fminf(fmaxf(rintf(v[4 + e] * g.out_inv_scale), -127.0f), 127.0f);
          lo |= (uint32_t)(q0 & 0xff) << (8 * e);
          hi |= (uint32_t)(q1 & 0xff) << (8 * e);
        }
        store(reinterpret_cast<uint2*>(op), make_uint2(lo, hi));
      } else {
#pragma unroll
        for (int h = 0; h < NV / 4; ++h)
          store(reinterpret_cast<float4*>(op) + h, make_float4(v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]));
      }
    }
  }
}

template <class TL, int ACT, bool RES, class TOUT, class TIN = bf16, class TW = TIN, bool RS = false>
int launch(const GemmArgs& g, hipStream_t stream) {
  const int64_t gy = cdiv(g.M, TL::BM), gx = cdiv(g.N, TL::BN);
  if (gy > 65535 || gx * gy > 0x7fffffffLL) return 0;
  hipLaunchKernelGGL((gemm_bf16_kernel<TL, ACT, RES, TOUT, TIN, TW, RS>), dim3((unsigned)gx, (unsigned)gy),
                     dim3(TL::THREADS), 0, stream, g);
  CORTEX_CHECK_LAUNCH("gemm_bf16_kernel");
  return 1;
}

using B128x128s2 = BTile<128, 128, 2, 2, 2>;
using B256x128s3 = BTile<256, 128, 3, 4, 2>;
using B256x256s2 = BTile<256, 256, 2, 4, 2>;
using B256x192s2 = BTile<256, 192, 2, 4, 2>;
using B128x128s2k2 = BTile<128, 128, 2, 2, 2, 2>;
// int8 weights widened at the fragment read: wavefronts span more rows, so that each widened
// W fragment feeds more MFMAs (128 x 64 and 128 x 32 wavefront tiles).  Measured at the
// forward's shapes: MLP-up 25.7 against 28.6 us with the bf16 tiles' layout, MLP-down 28.3
// against 30.2 us; the bf16 weights gain nothing from these layouts (22.9 / 25.4 us).
using B256x256s2w = BTile<256, 256, 2, 2, 4>;
using B128x128s2k2w = BTile<128, 128, 2, 1, 4, 2>;

int cu_count() {
  static int v = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return v;
}

// ---------------------------------------------------------------------------------------
// Persistent 256 x 256 tiles for bf16-output GEMMs past one wave of tiles (MLP-up with its
// GELU and the kv projection at B >= 64; bf16 rows and bf16 weight rows, N % 256 == 0).
//
// One workgroup per CU walks its tiles in turn (the tiles of an XCD in contiguous order, so
// the row panels stay shared in its L2).  When a tile's K loop is done, the workgroup first
// issues the next tile's first ring stages and only then runs the epilogue: the cold operand
// fetch of the next tile hides behind the GELU work, and the output stores drain while the
// next tile's first K steps run.  Launched as separate workgroups, each tile would pay both.
// The K loop, ring, swizzles and epilogue arithmetic are gemm_bf16_kernel's (B256x256s2,
// interleaved W rows, 8 consecutive columns per lane; transfers from a uniform base plus a
// 32-bit lane offset).  A tile's 256 column scales and biases travel into LDS with its first
// stages (two buffers, by tile parity, since the next tile's arrive during this tile's
// epilogue).  The epilogue issues exactly one 16-byte store per (row group, column group) and
// lane -- rows past M store row M - 1's values again, computed from the clamped A rows, so the
// duplicates are bit-identical -- so the first waits of the next tile count them exactly.
template <int ACT>
__global__ __launch_bounds__(512) void gemm_persist_kernel(GemmArgs g) {
  using TL = BTile<256, 256, 2, 4, 2>;
  using OP = Operand<bf16>;
  typedef OP::frag frag;
  constexpr int BM = TL::BM, BN = TL::BN, TM = TL::TM, TN = TL::TN, S = TL::STAGES;
  constexpr int AB = TL::A_BLOCKS, WB = TL::W_BLOCKS, PER = TL::PER;
  constexpr int NG = TN / 2;    // 8-column groups per lane
  constexpr int NST = TM * NG;  // stores per lane and tile
  static_assert(S == 2 && TL::KS == 1 && TL::WAVES == 8, "two-stage ring, one K group, 8 wavefronts");
  static_assert(PER + NST < 64, "vmcnt range");
  constexpr int PAR = TL::LDS;  // column parameters: [parity][scale 256 | bias 256] floats
  __shared__ __attribute__((aligned(1024))) unsigned char smem[TL::LDS + 2 * 2 * BN * 4];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / TL::WN, wn = wid % TL::WN;
  const int M = (int)g.M, K = (int)g.K;
  const int gx = (int)(g.N / BN), ntiles = (int)cdiv(g.M, (int64_t)BM) * gx;
  // tile order: XCD x (workgroups x, x + 8, ...) owns the contiguous eighth of the tiles
  const int G = gridDim.x;
  int t0, tstep, tend;
  if ((ntiles & 7) == 0 && (G & 7) == 0) {
    const int per_xcd = ntiles >> 3;
    t0 = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    tstep = G >> 3;
    tend = (blockIdx.x & 7) * per_xcd + per_xcd;
  } else {
    t0 = blockIdx.x;
    tstep = G;
    tend = ntiles;
  }
  const bf16* const A = reinterpret_cast<const bf16*>(g.x);
  const bf16* const W = reinterpret_cast<const bf16*>(g.w);
  const float* const scale = g.w_scale;
  const float* const bias = reinterpret_cast<const float*>(g.bias);
  // the LDS address of smem (wave-uniform) and of each wavefront's transfer blocks
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)smem);
  const int wu = __builtin_amdgcn_readfirstlane(wid);
  auto a_stage = [&](int s) __attribute__((always_inline)) { return smem + s * TL::A_STAGE; };
  auto w_stage = [&](int s) __attribute__((always_inline)) { return smem + S * TL::A_STAGE + s * TL::W_STAGE; };
  auto params = [&](int t) __attribute__((always_inline)) { return reinterpret_cast<float*>(smem + PAR) + (t & 1) * 2 * BN; };
  const int nk = K / TL::BK;

  // The transfer offsets (bytes from the operand bases; the host keeps both below 4 GiB) are
  // computed where the transfers are issued, from the tile's row and column origin, so that
  // no per-tile offsets stay live through the K loop and the epilogue.
  const int ldx = (int)g.ld_x, ldw = (int)g.ld_w;
  int m0c = 0, n0c = 0;  // origin of the tile whose transfers issue() sends
  auto issue = [&](int kt) __attribute__((always_inline)) {
    const int s = kt % S, k0 = kt * TL::BK;
    // the lane id through an instruction the compiler may not move: the offsets below are
    // recomputed at each issue instead of being kept live (or spilled) between issues
    int lane;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
#pragma unroll
    for (int i = 0; i < AB; ++i) {
      const int r = (wid * AB + i) * 8 + (lane >> 3);
      const uint32_t vo = (uint32_t)(min(m0c + r, M - 1) * ldx + ((lane & 7) ^ swz_a(r)) * 8) * 2u;
      lds_dma_m0<16>(A + k0, vo, lds0 + s * TL::A_STAGE + (wu * AB + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < WB; ++i) {
      const int r = (wid * WB + i) * 8 + (lane >> 3);
      const uint32_t vo = (uint32_t)((n0c + r) * ldw + ((lane & 7) ^ swz_w(r)) * 8) * 2u;
      lds_dma_m0<16>(W + k0, vo, lds0 + S * TL::A_STAGE + s * TL::W_STAGE + (wu * WB + i) * 1024);
    }
  };
  // a tile's first stages, its column parameters ahead of them (4 bytes per lane: wavefronts
  // 0-3 the 256 scales, 4-7 the biases; null ones are never read)
  auto prologue = [&](int t) __attribute__((always_inline)) {
    m0c = (t / gx) * BM;
    n0c = (t % gx) * BN;
    const int n0 = n0c;
    const float* src = wu < 4 ? scale : bias;
    if (src)
      lds_dma_m0<4>(src + n0 + (wu & 3) * 64, (uint32_t)(threadIdx.x & 63) * 4u,
                    lds0 + PAR + ((t & 1) * 2 * BN + (wu < 4 ? 0 : BN) + (wu & 3) * 64) * 4);
#pragma unroll
    for (int p = 0; p < S; ++p)
      if (p < nk) issue(p);
  };

  const int fr = lane & 15, g4 = lane >> 4;
  const int wrow = wm * (BM / TL::WM), wcol = wn * (BN / TL::WN);
  // Fragment reads: fragment t of A is row wrow + 16 t + fr and of W row wcol + wrow_of(t / 2,
  // t % 2, fr); their chunk swizzles depend on fr only (the tile offsets are multiples of 16
  // rows), so each sub-step's reads are one per-lane address plus compile-time offsets.
  const int a_x0 = (wrow + fr) * 128, w_x0 = (wcol + wrow_of(0, 0, fr)) * 128;
  const int a_sw0 = swz_a(fr), w_sw0 = swz_w(wrow_of(0, 0, fr));
  auto read_frags = [&](int stage, int ks, frag (&af)[TM], frag (&wf)[TN]) __attribute__((always_inline)) {
    const unsigned char* as = a_stage(stage) + a_x0 + (((ks * 4 + g4) ^ a_sw0) << 4);
    const unsigned char* ws = w_stage(stage) + w_x0 + (((ks * 4 + g4) ^ w_sw0) << 4);
#pragma unroll
    for (int t = 0; t < TM; ++t) af[t] = *reinterpret_cast<const frag*>(as + t * 16 * 128);
#pragma unroll
    for (int t = 0; t < TN; ++t)
      wf[t] = *reinterpret_cast<const frag*>(ws + (wrow_of(t >> 1, t & 1, 0)) * 128);
  };
  OP::accum acc[TM][TN];
  auto mma = [&](const frag (&af)[TM], const frag (&wf)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = OP::mma(wf[j], af[i], acc[i][j]);
  };
  bf16* const out = reinterpret_cast<bf16*>(g.out);

  frag af0[TM], af1[TM], wf0[TN], wf1[TN];
  // One K step handing over to the next, gemm_bf16_kernel's; `first_x`: step 0 of a tile whose
  // predecessor's NST epilogue stores were issued after this tile's first stages
  auto step = [&](int kt, auto refill, bool first_x) __attribute__((always_inline)) {
    const int st = kt % S;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): sub-step 0's fragments
    read_frags(st, 1, af1, wf1);
    __builtin_amdgcn_sched_barrier(0);
    mma(af0, wf0);
    __builtin_amdgcn_sched_barrier(0);
    // step kt + 1 landed: issued with the tile's first stages (only the stores are newer) or
    // in step kt - 1 (nothing newer)
    if (first_x)
      wait_vm<NST>();
    else
      wait_vm<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    read_frags((kt + 1) % S, 0, af0, wf0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (decltype(refill)::value) issue(kt + S);
    mma(af1, wf1);
  };

  // tile t's epilogue from registers and its column parameters in LDS: one store per (row
  // group, column group) and lane
  auto epilogue = [&](int t) __attribute__((always_inline)) {
    const int m0 = (t / gx) * BM, n0 = (t % gx) * BN;
    const float* sp = params(t);
    // row offsets in elements, 32-bit (M * ld_out * 2 < 4 GiB, checked at launch), once per tile
    uint32_t roff[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) roff[i] = (uint32_t)min(m0 + wrow + i * 16 + fr, M - 1) * (uint32_t)g.ld_out;
#pragma unroll
    for (int p = 0; p < NG; ++p) {
      const int c = wcol + 32 * p + 8 * g4;  // column inside the tile
      float sc[8], bi[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 s4 = *reinterpret_cast<const float4*>(sp + c + 4 * h);
        const float4 b4 = *reinterpret_cast<const float4*>(sp + BN + c + 4 * h);
        sc[4 * h] = scale ? s4.x : 1.f; sc[4 * h + 1] = scale ? s4.y : 1.f;
        sc[4 * h + 2] = scale ? s4.z : 1.f; sc[4 * h + 3] = scale ? s4.w : 1.f;
        bi[4 * h] = bias ? b4.x : 0.f; bi[4 * h + 1] = bias ? b4.y : 0.f;
        bi[4 * h + 2] = bias ? b4.z : 0.f; bi[4 * h + 3] = bias ? b4.w : 0.f;
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        bf16x8 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v0 = acc[i][2 * p][r] * sc[r] + bi[r];
          float v1 = acc[i][2 * p + 1][r] * sc[4 + r] + bi[4 + r];
          if constexpr (ACT == ACT_GELU) {
            v0 = gelu_erf_bf16out(v0);
            v1 = gelu_erf_bf16out(v1);
          }
          o[r] = (bf16)v0;
          o[4 + r] = (bf16)v1;
        }
        *reinterpret_cast<bf16x8*>(out + (roff[i] + (uint32_t)(n0 + c))) = o;
      }
    }
  };

  if (t0 >= tend) return;
  prologue(t0);
  bool after = false;  // the previous tile's epilogue stores are still counted by vmcnt
  for (int t = t0;; t += tstep) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = (OP::accum){0, 0, 0, 0};
    // step 0 landed (and the column parameters, issued before it)
    if (after) {
      if (nk > 1)
        wait_vm<PER + NST>();
      else
        wait_vm<NST>();
    } else {
      if (nk > 1)
        wait_vm<PER>();
      else
        wait_vm<0>();
    }
    __builtin_amdgcn_s_barrier();
    read_frags(0, 0, af0, wf0);
    int kt = 0;
    for (; kt + S < nk; ++kt) step(kt, std::integral_constant<bool, true>{}, after && kt == 0);
    for (; kt + 1 < nk; ++kt) step(kt, std::integral_constant<bool, false>{}, after && kt == 0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the last step
    read_frags((nk - 1) % S, 1, af1, wf1);
    mma(af0, wf0);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    mma(af1, wf1);
    const int next = t + tstep;
    __builtin_amdgcn_s_barrier();  // every wave is done with the ring: the next tile may refill it
    if (next < tend) prologue(next);
    epilogue(t);
    if (next >= tend) break;
    after = true;
  }
}

template <int ACT>
int launch_persist(const GemmArgs& g, hipStream_t stream) {
  const int64_t ntiles = cdiv(g.M, 256) * (g.N / 256);
  // 32-bit transfer offsets (the scalar-base form) address both operands, 32-bit element
  // offsets the output; larger tensors take the one-tile-per-workgroup kernel
  if (g.M * g.ld_x * 2 >= (1LL << 32) || g.N * g.ld_w * 2 >= (1LL << 32) || g.M * g.ld_out * 2 >= (1LL << 32) ||
      ntiles > 0x7fffffffLL)
    return 0;
  const int G = (int)std::min<int64_t>(ntiles, cu_count() & ~7);
  hipLaunchKernelGGL((gemm_persist_kernel<ACT>), dim3((unsigned)G), dim3(512), 0, stream, g);
  CORTEX_CHECK_LAUNCH("gemm_persist_kernel");
  return 1;
}

// ---------------------------------------------------------------------------------------
// Direct-weight residual GEMM: out = res + (A . W^T) * w_scale + bias (fp32; out may be res),
// A bf16 rows, W bf16 in MFMA fragment order (cortex_frag_weight), 128 x 128 tiles (MLP-down
// while the grid is at most one tile per CU).  Eight wavefronts in two K groups, each group
// taking half of K; wavefront (kg, wn) owns output columns 32 wn .. +31 of the tile for all 128
// rows, so no other wavefront reads its weight fragments: each is one contiguous 1 KiB read
// straight into the lane's operand registers, issued a K step ahead of its MFMAs, never staged
// in LDS.  The activation rows, which the four wavefronts of a group share, stream through a
// four-stage LDS ring per group with one barrier per two K steps (forward at B = 32 0.663-0.666
// -> 0.655-0.659 ms against two stages and a barrier per step, same box).  After the loop
// the groups swap halves of their partial tiles through LDS and each finishes 64 rows (their
// residual prefetched before the loop): per element the two K halves' sums are added once, as
// in the K-split tiles of gemm_bf16_kernel, with the same MFMA sequence per half, so the
// results equal that kernel's.
constexpr int RD_BM = 128, RD_BN = 128;

// NK = K / 128 (64-deep K steps per group), fully unrolled so that every wait is exact: across a
// loop's back edge the compiler cannot track the weight loads in flight and waits for all of
// them.  The activation rows go global -> VGPRs -> LDS (plain loads and ds_write) rather than by
// direct-to-LDS transfers: with those in flight the compiler's vmcnt count for the weight
// registers is no longer exact and it waits for every load (measured in its assembly).
template <int NK>
__global__ __launch_bounds__(512) void gemm_res_dw_kernel(GemmArgs g) {
  using OP = Operand<bf16>;
  typedef typename OP::frag frag;
  constexpr int TM = RD_BM / 16, TN = 2, HM = TM / 2;       // row tiles, column tiles, rows finished
  constexpr int A_STAGE = RD_BM * 128, AB = A_STAGE / 1024 / 4;  // 16 KiB; 4 chunks per lane and step
  constexpr int RS = 4;                                          // ring stages per K group
  constexpr int RING = RS * A_STAGE;
  constexpr int XCH = 8 * HM * TN * 64 * 16;                     // swapped half tiles
  constexpr int LDS = 2 * RING > XCH ? 2 * RING : XCH;
  static_assert(NK >= 2, "two K steps per group at least");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[LDS];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int kg = wid >> 2, wn = wid & 3;
  const int fr = lane & 15, g4 = lane >> 4;
  const int nbx = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + nbx * blockIdx.y, total);  // contiguous row tiles per XCD
  const int m0 = (id / nbx) * RD_BM, n0 = (id % nbx) * RD_BN;
  const int M = (int)g.M;
  constexpr int K = NK * 128;
  const int kb = kg * (K / 2);  // the group's first K
  unsigned char* const ring = smem + kg * RING;

  // activation chunks: block q = 4 wn + i of a stage holds rows 8 q .. +7; lane l's 16 bytes
  // are row 8 q + l / 8, logical chunk (l % 8) ^ swz_a(row), stored at byte 16 l of the block
  const bf16* a_src[AB];
#pragma unroll
  for (int i = 0; i < AB; ++i) {
    const int r = (wn * AB + i) * 8 + (lane >> 3);
    a_src[i] = reinterpret_cast<const bf16*>(g.x) + (int64_t)min(m0 + r, M - 1) * g.ld_x + kb +
               ((lane & 7) ^ swz_a(r)) * 8;
  }
  unsigned char* const a_dst = ring + wn * AB * 1024 + lane * 16;
  frag ar[NK][AB];  // (fully unrolled: registers of their own per step)
  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < AB; ++i) ar[kt][i] = *reinterpret_cast<const frag*>(a_src[i] + kt * 64);
  };
  auto store_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < AB; ++i) *reinterpret_cast<frag*>(a_dst + (kt % RS) * A_STAGE + i * 1024) = ar[kt][i];
  };
  // weight fragment (t, ks) of step kt: block ((n0 + 32 wn) / 16 + t, kb / 32 + 2 kt + ks), this lane's 16 bytes
  const bf16* wp = reinterpret_cast<const bf16*>(g.w) + ((int64_t)((n0 + 32 * wn) / 16) * (K / 32) + kb / 32) * 512 +
                   lane * 8;
  frag wb[NK][TN][2];
  auto load_w = [&](int kt) {
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        wb[kt][t][ks] = *reinterpret_cast<const frag*>(wp + (t * (K / 32) + 2 * kt + ks) * 512);
  };

  typename OP::accum acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (typename OP::accum){0, 0, 0, 0};
  const int a_row = fr * 128, a_sw = swz_a(fr);  // rows 16 t + fr: the same swizzle for every t
  auto read_a = [&](int st, int ks, frag (&af)[TM]) {
    const unsigned char* as = ring + st * A_STAGE + a_row + (((ks * 4 + g4) ^ a_sw) << 4);
#pragma unroll
    for (int t = 0; t < TM; ++t) af[t] = *reinterpret_cast<const frag*>(as + t * 2048);
  };
  auto mma = [&](const frag (&af)[TM], int kt, int ks) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = OP::mma(wb[kt][j][ks], af[i], acc[i][j]);
  };

  // issue order: A(0..2), W(0), W(1), the residual of the rows this group finishes.  The ring has
  // four stages and a barrier after every second step: in step kt, A(kt + 2) goes from registers
  // into its stage (read last in step kt - 2, before the previous barrier), A(kt + 3) into
  // registers, and after the MFMAs W(kt + 2); the barrier closing steps kt and kt + 1 publishes
  // the stages of kt + 2 and kt + 3, so the wavefronts of a workgroup may drift apart by a step
  load_a(0);
  load_a(1);
  if (NK > 2) load_a(2);
  load_w(0);
  load_w(1);
  const float* res = reinterpret_cast<const float*>(g.res);
  const int res_rows = g.res_rows > 0 ? (int)g.res_rows : M;
  float4 rv[HM][TN];
#pragma unroll
  for (int ii = 0; ii < HM; ++ii) {
    const int m = min(m0 + (kg * HM + ii) * 16 + fr, M - 1);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      rv[ii][j] = *reinterpret_cast<const float4*>(res + (int64_t)(m % res_rows) * g.ld_res + n0 + 32 * wn + 16 * j +
                                                   4 * g4);
  }
  store_a(0);
  store_a(1);
  __syncthreads();  // stages 0 and 1 of both groups written
  frag af0[TM], af1[TM];
  read_a(0, 0, af0);
#pragma unroll
  for (int kt = 0; kt < NK; ++kt) {
    const int st = kt % RS;
    __builtin_amdgcn_sched_barrier(0);
    read_a(st, 1, af1);
    mma(af0, kt, 0);
    if (kt + 2 < NK) store_a(kt + 2);
    if ((kt & 1) && kt + 1 < NK) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): these writes and this wave's reads of the pair's stages
      __builtin_amdgcn_s_barrier();        // every wave's: steps kt + 1, kt + 2 visible, the pair's stages free
    }
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < NK) read_a((kt + 1) % RS, 0, af0);
    if (kt + 3 < NK) load_a(kt + 3);
    mma(af1, kt, 1);
    if (kt + 2 < NK) load_w(kt + 2);
  }

  // swap halves through LDS: group kg finishes rows 16 (kg HM + ii) + fr and sends the others
  float4* xch = reinterpret_cast<float4*>(smem);
  const float* bias = reinterpret_cast<const float*>(g.bias);
  float* out = reinterpret_cast<float*>(g.out);
  auto finish = [&](auto half) {
    constexpr int own = decltype(half)::value, other = 1 - own;
    float4 sc[TN], bi[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + 32 * wn + 16 * j + 4 * g4;
      sc[j] = g.w_scale ? *reinterpret_cast<const float4*>(g.w_scale + n) : make_float4(1.f, 1.f, 1.f, 1.f);
      bi[j] = bias ? *reinterpret_cast<const float4*>(bias + n) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();  // every ring read is done: the exchange area may overwrite the rings
#pragma unroll
    for (int ii = 0; ii < HM; ++ii)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const typename OP::accum v = acc[other * HM + ii][j];
        xch[((wid * HM + ii) * TN + j) * 64 + lane] = make_float4(v[0], v[1], v[2], v[3]);
      }
    __syncthreads();
    const int partner = other * 4 + wn;
    wait_vm<0>();
    const WtOut store(out, (int64_t)M * g.ld_out * 4, wt_one_wave());
#pragma unroll
    for (int ii = 0; ii < HM; ++ii) {
      const int m = m0 + (own * HM + ii) * 16 + fr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        // the two K halves' sums added once (commutative: which group adds is of no concern)
        const float4 o = xch[((partner * HM + ii) * TN + j) * 64 + lane];
        const typename OP::accum a = acc[own * HM + ii][j];
        const float4 x = rv[ii][j];
        const float y0 = (a[0] + o.x) * sc[j].x + bi[j].x + x.x;
        const float y1 = (a[1] + o.y) * sc[j].y + bi[j].y + x.y;
        const float y2 = (a[2] + o.z) * sc[j].z + bi[j].z + x.z;
        const float y3 = (a[3] + o.w) * sc[j].w + bi[j].w + x.w;
        if (m < M) store(reinterpret_cast<float4*>(out + (int64_t)m * g.ld_out + n0 + 32 * wn + 16 * j + 4 * g4),
                         make_float4(y0, y1, y2, y3));
      }
    }
  };
  if (kg == 0) finish(std::integral_constant<int, 0>{});
  else finish(std::integral_constant<int, 1>{});
}

int launch_res_dw_impl(const GemmArgs& g, hipStream_t stream) {
  const int64_t gy = cdiv(g.M, (int64_t)RD_BM), gx = g.N / RD_BN;
  CORTEX_CHECK_ARG(gy <= 65535 && gx * gy <= 0x7fffffffLL, "gemm_res_dw_kernel: M=%lld exceeds the grid limit",
                   (long long)g.M);
  const dim3 grid((unsigned)gx, (unsigned)gy);
  switch (g.K) {
    case 1024: hipLaunchKernelGGL(gemm_res_dw_kernel<8>, grid, dim3(512), 0, stream, g); break;
    case 2048: hipLaunchKernelGGL(gemm_res_dw_kernel<16>, grid, dim3(512), 0, stream, g); break;
    case 3072: hipLaunchKernelGGL(gemm_res_dw_kernel<24>, grid, dim3(512), 0, stream, g); break;
    default:
      set_error("gemm_res_dw_kernel: K=%lld is not 1024, 2048 or 3072", (long long)g.K);
      return E_INVALID;
  }
  CORTEX_CHECK_LAUNCH("gemm_res_dw_kernel");
  return OK;
}

// Tile by shape: 256-row tiles halve the operand traffic per MFMA, so take the widest tile
// that still fills (nearly) every CU once, else 128 x 128 (two workgroups per CU).
enum TileChoice { T128 = 0, T256 = 4, T192 = 6, T128_K2 = 7 };
TileChoice wide_tile(const GemmArgs& g, bool allow192) {
  const int64_t t256 = cdiv(g.M, 256) * cdiv(g.N, 256), t192 = cdiv(g.M, 256) * cdiv(g.N, 192);
  const int ncu = cu_count();
  if (g.N % 256 == 0 && t256 >= ncu * 15 / 16) return T256;
  if (allow192 && g.N % 192 == 0 && t192 >= ncu * 15 / 16 && t192 <= ncu) return T192;
  if (t256 >= ncu * 3 / 4) return T256;
  return T128;
}

template <int ACT, bool RES, class TOUT, class TW = bf16>
int dispatch(const GemmArgs& g, hipStream_t stream) {
  if constexpr (sizeof(TW) == 1) {
    // int8 weights (widened at the fragment read): the same tiles as bf16 weights but the
    // 192-column one
    return wide_tile(g, false) == T256 ? launch<B256x256s2w, ACT, RES, TOUT, bf16, TW>(g, stream)
                                       : launch<B128x128s2, ACT, RES, TOUT, bf16, TW>(g, stream);
  } else {
    switch (wide_tile(g, true)) {
      case T256:
        // past one wave of 256 x 256 tiles, bf16 out: persistent tiles (see gemm_persist_kernel)
        if constexpr (!RES && sizeof(TOUT) == 2) {
          if (g.N % 256 == 0 && cdiv(g.M, 256) * (g.N / 256) > cu_count() && cu_count() >= 8) {
            const int st = launch_persist<ACT>(g, stream);
            if (st != 0) return st;
          }
        }
        return launch<B256x256s2, ACT, RES, TOUT>(g, stream);
      case T192: return launch<B256x192s2, ACT, RES, TOUT>(g, stream);
      default: return launch<B128x128s2, ACT, RES, TOUT>(g, stream);
    }
  }
}

// RMSNorm without a gain (the gain folded into bf16 weight rows): the plain GEMM, its A
// fragments also summed as squares, 1 / rms on the accumulator.  Tiles as dispatch() picks
// them for bf16 weights (256 x 256, 256 x 192, 128 x 128), and for grids of at most one
// 128 x 128 workgroup per CU the K split of the residual GEMMs.
template <int ACT, class TOUT>
int dispatch_rs(const GemmArgs& g, hipStream_t stream) {
  TileChoice t = wide_tile(g, true);
  // at most one 128 x 128 workgroup per CU: K split over two wave groups (eight wavefronts)
  if (t == T128 && g.K % 128 == 0 && cdiv(g.M, 128) * cdiv(g.N, 128) <= cu_count()) t = T128_K2;
  switch (t) {
    case T256: return launch<B256x256s2, ACT, false, TOUT, bf16, bf16, true>(g, stream);
    case T192: return launch<B256x192s2, ACT, false, TOUT, bf16, bf16, true>(g, stream);
    case T128_K2: return launch<B128x128s2k2, ACT, false, TOUT, bf16, bf16, true>(g, stream);
    default: return launch<B128x128s2, ACT, false, TOUT, bf16, bf16, true>(g, stream);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------------------------------
// Norm prologue + GEMM in one kernel (rms_norm_linear, reference cortex/kernels/
// fused_rmsnorm.py:130-233, and its INT8-weight / LayerNorm forms):
//
//   C[m, n] = epi( sum_k y[m, k] W[n, k] ),  y = bf16( x / sqrt(mean(x^2) + eps) * gamma )   (RMS)
//                                            y = bf16( (x - mu) / sqrt(var + eps) * gamma + beta ) (LN)
//
struct NormGemmArgs {
  int64_t M, N, K;
  const bf16* x;
  int64_t ld_x;
  int norm;  // NORM_RMS or NORM_LAYER
  const void* gamma;
  const void* beta;  // LayerNorm only (may be null)
  int gamma_dtype;   // DT_F32 or DT_BF16 (beta the same)
  float eps;
  const void* w;  // (N, K) rows: bf16 or int8
  int64_t ld_w;
  const float* w_scale;
  const float* bias;
  void* out;
  int64_t ld_out;
  int groups;  // G: column-tile groups per row panel (gridDim.x)
};

// Direct-to-LDS transfer of 16 bytes per lane (global_load_lds_dwordx4, LDS destination
// lds_dst + 16 * lane) issued from inline assembly, so that the compiler does not treat
// the LDS reads that follow as aliasing the transfer and wait for every transfer in
// flight (it cannot tell ring stages apart).  The kernel's own vmcnt waits and barriers
// order each stage's reads after its transfers; the compiler's waits for its own vector
// loads stay conservative, as it counts fewer operations in flight than there are.  A
// flat pointer to LDS carries the LDS offset in its low 32 bits (the aperture base is
// 4 GiB aligned).
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds_dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gsrc), "s"(m0) : "memory", "m0");
}

// Register-resident rows.  Eight wavefronts (two per SIMD) on a 128-row panel for all of
// K (K <= 512): wavefronts w and w + 4 share rows 32 (w % 4) .. + 31 and split every
// 64-column tile between them (columns 16 (l / 16) + 8 (w / 4) + [0, 8) of lane l).
// Each wavefront transfers half of its 32 rows into LDS (one 1 KiB row per transfer, full
// cache lines), reads them in the MFMA operand layout, computes their statistics (a lane's
// partial sums, then the four lanes that share a row), normalises them to bf16 in
// registers and writes them back; it then reads its partner's normalised half, so every
// row is normalised once per workgroup.  The rows stay in VGPRs while the workgroup walks
// its column tiles.  Lane l holds row l % 16 of each 16-row group and, of each 64-wide K
// step s, the slice 64 s + 16 (l / 16) + [0, 16): the two 8-value halves feed the two
// 32-deep MFMAs of the step, and the weight fragments are read with the same slice, so
// the contraction pairs the right k.  In the tile loop only the weight passes through
// LDS, as bf16 rows: one whole 64 x K tile per buffer, two buffers, one barrier per tile,
// the fragments of K step s + 1 read while step s multiplies.  A bf16 weight is
// transferred direct to LDS; an int8 weight is loaded into registers during the previous
// tile's multiplications, widened exactly and written as bf16 rows (once per workgroup).
// The first tile comes through registers (its loads overlap the normalisation, whose
// staging area the tile buffers reuse).  The tile's scales and biases ride along in a
// 1 KiB transfer.
//
// LDS rows (the staged x rows and the weight rows) are 1024 + 16 bytes apart, so the 16
// consecutive rows one fragment read touches start in 16 different four-bank groups and
// every read address is a per-lane base plus a compile-time offset.
//
// Output columns: LDS weight row 16 f + i (fragment f, fragment row i) holds column
// 16 (i / 4) + 8 (f / 2) + 4 (f % 2) + i % 4 of the tile, so lane l of wavefront w ends
// with the eight consecutive columns 16 (l / 16) + 8 (w / 4) + [0, 8) of its row (one
// 16-byte bf16 store).  Rows past M read row M - 1 and column groups past N read the last
// eight columns, so every lane computes a valid output and stores it: duplicates are
// bit-identical, and each tile issues a fixed number of stores, which the next tile's
// vmcnt wait counts exactly.
struct RTile {
  static constexpr int RG = 2, WAVES = 8, THREADS = 512, BM = 128, BN = 64, KMAX = 512;
  static constexpr int RP = KMAX * 2 + 16;  // LDS bytes from one bf16 row to the next
  static constexpr int W_TILE = BN * RP;
  static constexpr int XS = BM * RP;        // the panel's rows, staged once (aliases the tiles)
  static constexpr int SB = 1024, GB = 2 * KMAX * 4;
  static constexpr int BODY = XS > 2 * W_TILE ? XS : 2 * W_TILE;
  static constexpr int LDS = BODY + 2 * SB + GB;
  static_assert(LDS <= 160 * 1024 && 16 * 3 * RP + 128 * 7 + 16 < 65536, "LDS");
};

// global weight row held by LDS row R of the tile at column n0 (see the column order above)
__device__ __forceinline__ int rk_wrow(int R, int n0, int N) {
  const int f = R >> 4, i = R & 15;
  return min(n0 + 16 * (i >> 2) + 8 * (f >> 1), N - 8) + 4 * (f & 1) + (i & 3);
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): indices that are
// constants when the code is generated (register arrays indexed this way stay in VGPRs)
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int NORM, bool NRM, class TW, int ACT, class TOUT>
__global__ __launch_bounds__(512) void norm_gemm_rk_kernel(NormGemmArgs g) {
  using TL = RTile;
  constexpr int BN = TL::BN, RP = TL::RP;
  constexpr bool WI8 = sizeof(TW) == 1, OBF = sizeof(TOUT) == 2;
  constexpr int EPI = 2 * (OBF ? 1 : 2);  // global stores per lane per tile
  constexpr int NW0 = WI8 ? 4 : 8;        // 16-byte register loads per lane of one weight tile
  __shared__ __attribute__((aligned(1024))) unsigned char smem[TL::LDS];
  auto wbuf = [&](int b) { return smem + b * TL::W_TILE; };
  auto sbuf = [&](int b) { return smem + TL::BODY + b * TL::SB; };
  unsigned char* const gbuf = smem + TL::BODY + 2 * TL::SB;  // fp32 gamma at 0, beta at KMAX * 4

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int pr = wid & 3, c2 = wid >> 2;  // row pair (rows 32 pr ..) and column half
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K, nk = K / 64;
  // plain stores: wavefronts w and w + 4 write alternate 16-byte pieces of each 128-byte output
  // line, which the L2 merges; written through, each half crosses to memory on its own (twice
  // the write bytes, no time saved)
  const int G = gridDim.x, total = gridDim.x * gridDim.y;
  const int id = xcd_affine(blockIdx.x + G * blockIdx.y, total);
  const int m0 = (id / G) * TL::BM, grp = id % G;
  const int ntiles = (N + BN - 1) / BN;
  const int nt = grp < ntiles ? (ntiles - 1 - grp) / G + 1 : 0;
  if (nt == 0) return;  // uniform over the workgroup
  const int j16 = lane & 15, q = lane >> 4;
  const unsigned ldb = (unsigned)(g.ld_w * (int64_t)sizeof(TW));  // N * ldb < 2^31 (checked by the host)

  // the tile's scales and biases: lanes 0-15 scale, 16-31 bias, 4 columns each (wavefront 0)
  auto issue_sb = [&](int i, int b) {
    if (wid == 0) {
      const int n0 = (grp + i * G) * BN;
      const float* base = (lane & 16) ? g.bias : g.w_scale;
      const float* src = base ? base + min(n0 + 4 * (lane & 15), N - 4) : reinterpret_cast<const float*>(g.w);
      lds_dma16(src, sbuf(b));
    }
  };
  // bf16 weight direct to LDS: 8 rows (1 KiB each) per wavefront
  auto issue_w16 = [&](int i, int b) {
    const int n0 = (grp + i * G) * BN;
    const unsigned char* wl = reinterpret_cast<const unsigned char*>(g.w) + min(lane, K / 8 - 1) * 16;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int R = 8 * wid + t;
      lds_dma16(wl + (unsigned)rk_wrow(R, n0, N) * ldb, wbuf(b) + R * RP);
    }
  };
  // a weight tile through registers: bf16, one row per load (lane: 16-byte chunk); int8, two
  // rows per load (lane / 32 the row, lane % 32 the chunk of 16 values, widened on the store)
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  // two register sets (native vector types: a HIP uint4 array here ends up in scratch); the
  // int8 tile loop alternates them, widening one while the other is in flight
  u32x4 wr[NW0], wr2[NW0];
  auto wreg_row = [&](int t) { return WI8 ? 8 * wid + 2 * t + (lane >> 5) : 8 * wid + t; };
  auto load_wreg = [&](int i, u32x4 (&w)[NW0]) {
    const int n0 = (grp + i * G) * BN;
    const int c = WI8 ? min(lane & 31, K / 16 - 1) : min(lane, K / 8 - 1);
    const unsigned char* wl = reinterpret_cast<const unsigned char*>(g.w) + c * 16;
    static_for<NW0>([&](auto t) {
      w[t] = *reinterpret_cast<const u32x4*>(wl + (unsigned)rk_wrow(wreg_row(t), n0, N) * ldb);
    });
  };
  // load t of a register set into buffer b (int8: widened exactly)
  auto store_piece = [&](int b, const u32x4 (&wr)[NW0], auto tc) {
    constexpr int t = decltype(tc)::value;
    {
      unsigned char* d = wbuf(b) + wreg_row(t) * RP;
      if constexpr (WI8) {
        d += (lane & 31) * 32;
        *reinterpret_cast<bf16x8*>(d) = widen_i8x8(make_uint2(wr[t][0], wr[t][1]));
        *reinterpret_cast<bf16x8*>(d + 16) = widen_i8x8(make_uint2(wr[t][2], wr[t][3]));
      } else {
        *reinterpret_cast<u32x4*>(d + lane * 16) = wr[t];
      }
    }
  };
  auto store_wreg = [&](int b, const u32x4 (&w)[NW0]) { static_for<NW0>([&](auto t) { store_piece(b, w, t); }); };

  // ---- prologue: tile 0's weight into registers and its scales into LDS, this wavefront's
  // 16 rows (rows 32 pr + 16 c2 ..) into LDS, gamma / beta (int8: tile 1's weight as well)
  load_wreg(0, wr);
  if constexpr (WI8) load_wreg(1, wr2);
  issue_sb(0, 0);
  const int own = 32 * pr + 16 * c2;  // first staged row of this wavefront
  {
    const bf16* xl = g.x + min(lane, K / 8 - 1) * 8;
#pragma unroll
    for (int t = 0; t < 16; ++t) lds_dma16(xl + (int64_t)min(m0 + own + t, M - 1) * g.ld_x, smem + (own + t) * RP);
    // gamma / beta: fp32 straight into gbuf; bf16 into tile 1's scale area, widened below
    const bool gbf = g.gamma_dtype == DT_BF16;
    const int esz = gbf ? 2 : 4;
    const int nb = esz * TL::KMAX / 1024;  // 1 KiB blocks per vector: 1 or 2
    if (NRM && wid < 2 * nb) {
      const int which = wid / nb, blk = wid % nb;
      const void* base = (which && g.beta) ? g.beta : g.gamma;
      const int c = min(blk * 64 + lane, K * esz / 16 - 1);
      unsigned char* dst = gbf ? sbuf(1) + which * 1024 : gbuf + which * (TL::KMAX * 4) + blk * 1024;
      lds_dma16(reinterpret_cast<const unsigned char*>(base) + c * 16, dst);
    }
  }
  wait_vm<0>();  // this wavefront's rows, tile 0's weight and scales, its gamma / beta block
  // a[0]: this wavefront's own 16 rows (normalised here when NRM), a[1]: its partner's 16 rows
  const int other = 32 * pr + 16 * (1 - c2);
  bf16x8 a[2][8][2];
  const unsigned char* xo = smem + (own + j16) * RP + 32 * q;
  bf16x8 (&mine)[8][2] = a[0];
  float rinv[2] = {1.0f, 1.0f};  // without NRM: 1 / rms of this lane's row in a[0], a[1]
  if constexpr (NRM) {
    {
      bf16x8 (&v)[8][2] = mine;  // raw rows, normalised in place
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) v[s][h] = *reinterpret_cast<const bf16x8*>(xo + s * 128 + h * 16);
      // statistics: a lane's partial sums over its 8 x 16 values, then the four lanes of the
      // row (l, l ^ 16, l ^ 32, l ^ 48)
      const float fk = (float)K;  // means as sum / K, as torch's mean
      const bf16x2_t ones = {(__bf16)1.0f, (__bf16)1.0f};
      float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (s < nk) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const bf16x2_t xv = pair_of(v[s][h], d);
              // sum of squares (RMS) or sum (LayerNorm): bf16 products are exact in fp32
              p[d] = __builtin_amdgcn_fdot2_f32_bf16(xv, NORM == NORM_RMS ? xv : ones, p[d], false);
            }
        }
      }
      float s1 = (p[0] + p[1]) + (p[2] + p[3]);
      s1 += __shfl_xor(s1, 16, 64);
      s1 += __shfl_xor(s1, 32, 64);
      float mu = 0.0f, inv;
      if constexpr (NORM == NORM_RMS) {
        inv = 1.0f / sqrtf(s1 / fk + g.eps);
      } else {
        mu = s1 / fk;
        float s2[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if (s < nk) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float d0 = (float)v[s][h][e] - mu;
                s2[e & 3] = fmaf(d0, d0, s2[e & 3]);
              }
          }
        }
        float t2 = (s2[0] + s2[1]) + (s2[2] + s2[3]);
        t2 += __shfl_xor(t2, 16, 64);
        t2 += __shfl_xor(t2, 32, 64);
        inv = 1.0f / sqrtf(t2 / fk + g.eps);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();  // gamma / beta of every wavefront landed
      if (g.gamma_dtype == DT_BF16) {
        for (int e = tid; e < 2 * TL::KMAX; e += TL::THREADS)
          reinterpret_cast<float*>(gbuf)[e] = (float)reinterpret_cast<const bf16*>(sbuf(1))[e];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
      }
      // normalise: y = bf16((x - mu) inv gamma + beta); K steps past K are 0; back to LDS
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (s < nk) {
          float gm[16], bt[16];
          const unsigned char* gp = gbuf + (64 * s + 16 * q) * 4;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float4 g4 = *reinterpret_cast<const float4*>(gp + 16 * c);
            gm[4 * c] = g4.x; gm[4 * c + 1] = g4.y; gm[4 * c + 2] = g4.z; gm[4 * c + 3] = g4.w;
            if constexpr (NORM != NORM_RMS) {
              const float4 b4 = *reinterpret_cast<const float4*>(gp + TL::KMAX * 4 + 16 * c);
              const bool hb = g.beta != nullptr;
              bt[4 * c] = hb ? b4.x : 0.0f;
              bt[4 * c + 1] = hb ? b4.y : 0.0f;
              bt[4 * c + 2] = hb ? b4.z : 0.0f;
              bt[4 * c + 3] = hb ? b4.w : 0.0f;
            }
          }
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float xv = (float)v[s][h][e];
              if constexpr (NORM == NORM_RMS)
                mine[s][h][e] = (bf16)((xv * inv) * gm[8 * h + e]);
              else
                mine[s][h][e] = (bf16)fmaf((xv - mu) * inv, gm[8 * h + e], bt[8 * h + e]);
            }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) mine[s][h][e] = (bf16)0.0f;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) *reinterpret_cast<bf16x8*>(const_cast<unsigned char*>(xo) + s * 128 + h * 16) = mine[s][h];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // every wavefront's normalised rows in LDS
    {
      bf16x8 (&theirs)[8][2] = a[1];
      const unsigned char* xp = smem + (other + j16) * RP + 32 * q;
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) theirs[s][h] = *reinterpret_cast<const bf16x8*>(xp + s * 128 + h * 16);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // the staged rows are dead: the tile buffers may overwrite them
  } else {
    // rows as given (the gain is in the weight): both halves straight from LDS, the
    // statistics of both, and 1 / rms applied to the accumulator in the epilogue
    __builtin_amdgcn_s_barrier();  // the partner's rows landed
    const unsigned char* xp = smem + (other + j16) * RP + 32 * q;
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        a[0][s][h] = *reinterpret_cast<const bf16x8*>(xo + s * 128 + h * 16);
        a[1][s][h] = *reinterpret_cast<const bf16x8*>(xp + s * 128 + h * 16);
      }
    const float fk = (float)K;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (s < nk) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const bf16x2_t xv = pair_of(a[r][s][h], d);
              p[d] = __builtin_amdgcn_fdot2_f32_bf16(xv, xv, p[d], false);
            }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) a[r][s][h] = (bf16x8){};  // K steps past K are 0
        }
      }
      float s1 = (p[0] + p[1]) + (p[2] + p[3]);
      s1 += __shfl_xor(s1, 16, 64);
      s1 += __shfl_xor(s1, 32, 64);
      rinv[r] = 1.0f / sqrtf(s1 / fk + g.eps);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // the staged rows are dead: the tile buffers may overwrite them
  }
  store_wreg(0, wr);

  // ---- epilogue of one tile: scale, bias (from the tile's LDS copy), activation, stores
  auto epilogue = [&](const f32x4 (&ac)[2][2], int n0, int sbi) {
    const unsigned char* sb = sbuf(sbi);
    const int cs = min(n0 + 16 * q + 8 * c2, N - 8), lc = cs - n0;
    float sc[8], bi[8];
    {
      const float4 s0 = *reinterpret_cast<const float4*>(sb + 4 * lc), s1 = *reinterpret_cast<const float4*>(sb + 4 * lc + 16);
      const float4 b0 = *reinterpret_cast<const float4*>(sb + 256 + 4 * lc), b1 = *reinterpret_cast<const float4*>(sb + 256 + 4 * lc + 16);
      const bool hs = g.w_scale != nullptr, hb = g.bias != nullptr;
      sc[0] = hs ? s0.x : 1.f; sc[1] = hs ? s0.y : 1.f; sc[2] = hs ? s0.z : 1.f; sc[3] = hs ? s0.w : 1.f;
      sc[4] = hs ? s1.x : 1.f; sc[5] = hs ? s1.y : 1.f; sc[6] = hs ? s1.z : 1.f; sc[7] = hs ? s1.w : 1.f;
      bi[0] = hb ? b0.x : 0.f; bi[1] = hb ? b0.y : 0.f; bi[2] = hb ? b0.z : 0.f; bi[3] = hb ? b0.w : 0.f;
      bi[4] = hb ? b1.x : 0.f; bi[5] = hb ? b1.y : 0.f; bi[6] = hb ? b1.z : 0.f; bi[7] = hb ? b1.w : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int m = min(m0 + (r ? other : own) + j16, M - 1);
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (NRM) {
          v[e] = ac[r][0][e] * sc[e] + bi[e];
          v[4 + e] = ac[r][1][e] * sc[4 + e] + bi[4 + e];
        } else {
          v[e] = (ac[r][0][e] * rinv[r]) * sc[e] + bi[e];
          v[4 + e] = (ac[r][1][e] * rinv[r]) * sc[4 + e] + bi[4 + e];
        }
      }
      if (ACT == ACT_GELU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = OBF ? gelu_erf_bf16out(v[e]) : gelu_erf(v[e]);
      }
      TOUT* op = reinterpret_cast<TOUT*>(g.out) + (int64_t)m * g.ld_out + cs;
      if constexpr (OBF) {
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (bf16)v[e];
        *reinterpret_cast<bf16x8*>(op) = o;
      } else {
        *reinterpret_cast<float4*>(op) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(op + 4) = make_float4(v[4], v[5], v[6], v[7]);
      }
    }
  };

  // ---- column tiles.  int8: during tile i the registers `cur` hold tile i + 1's rows (loaded
  // a tile earlier), widened piece by piece between the K steps into the other buffer, while
  // `nxt` receives tile i + 2's (the last tiles' successors clamp into range; their buffer is
  // never read).  bf16: tile i + 1 is transferred direct to LDS at the top of tile i.
  auto tile = [&](int i, const u32x4 (&cur)[NW0], u32x4 (&nxt)[NW0]) {
    const int n0 = (grp + i * G) * BN, b = i & 1;
    if (i > 0) {
      if constexpr (WI8)
        wait_vm<NW0 + EPI>();  // tile i's scales: issued before tile i + 1's loads and tile i - 1's stores
      else
        wait_vm<EPI>();  // tile i's transfers: only the previous tile's stores were issued after them
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's LDS reads and writes done
    __builtin_amdgcn_s_barrier();        // tile i visible; buffer b ^ 1 free (tile i - 1 done)
    if constexpr (WI8) {
      issue_sb(i + 1, b ^ 1);
      load_wreg(i + 2, nxt);
    } else if (i + 1 < nt) {
      issue_sb(i + 1, b ^ 1);
      issue_w16(i + 1, b ^ 1);
    }

    const unsigned char* wb = wbuf(b) + (32 * c2 + j16) * RP + 32 * q;  // fragments 2 c2, 2 c2 + 1
    f32x4 acc[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int f = 0; f < 2; ++f) acc[r][f] = (f32x4){0, 0, 0, 0};
    bf16x8 cf[2][2], nf[2][2];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int h = 0; h < 2; ++h) cf[f][h] = *reinterpret_cast<const bf16x8*>(wb + f * 16 * RP + h * 16);
    static_for<8>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      if constexpr (s + 1 < 8) {
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            nf[f][h] = *reinterpret_cast<const bf16x8*>(wb + f * 16 * RP + (s + 1) * 128 + h * 16);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int r = 0; r < 2; ++r)
            acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cf[f][h], a[r][s][h], acc[r][f], 0, 0, 0);
      if constexpr (WI8 && s < NW0) store_piece(b ^ 1, cur, std::integral_constant<int, s>{});
      if constexpr (s + 1 < 8) {
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int h = 0; h < 2; ++h) cf[f][h] = nf[f][h];
      }
    });
    epilogue(acc, n0, b);
  };
  for (int i = 0; i < nt; i += 2) {
    tile(i, wr2, wr);
    if (i + 1 < nt) tile(i + 1, wr, wr2);
  }
}

template <int NORM, bool NRM, class TW, int ACT, class TOUT>
int launch_norm_rk(const NormGemmArgs& a0, hipStream_t stream) {
  using TL = RTile;
  NormGemmArgs a = a0;
  const int64_t panels = cdiv(a.M, TL::BM), ntiles = cdiv(a.N, TL::BN);
  // column-tile groups: one workgroup per CU
  int64_t G = cdiv((int64_t)cu_count(), panels);
  G = G < 1 ? 1 : (G > ntiles ? ntiles : G);
  if (panels > 65535 || G * panels > 0x7fffffffLL) return 0;
  a.groups = (int)G;
  hipLaunchKernelGGL((norm_gemm_rk_kernel<NORM, NRM, TW, ACT, TOUT>), dim3((unsigned)G, (unsigned)panels), dim3(TL::THREADS),
                     0, stream, a);
  CORTEX_CHECK_LAUNCH("norm_gemm_rk_kernel");
  return 1;
}

template <class TW, int ACT, class TOUT>
int dispatch_norm(const NormGemmArgs& a, hipStream_t stream) {
  // rows normalised in the kernel (LayerNorm, RMS with a gain), or RMS without a gain: raw
  // rows and 1 / rms on the accumulator (cortex_fold_gain builds a weight that carries it;
  // a bf16 weight of that form goes to dispatch_rs while the rows stay below 4 GiB)
  if (a.norm == NORM_LAYER) return launch_norm_rk<NORM_LAYER, true, TW, ACT, TOUT>(a, stream);
  return a.gamma ? launch_norm_rk<NORM_RMS, true, TW, ACT, TOUT>(a, stream)
                 : launch_norm_rk<NORM_RMS, false, TW, ACT, TOUT>(a, stream);
}

}  // namespace

int split_k_partials(const GemmArgs& g, int splits, hipStream_t stream) {
  using TL = B128x128s2;
  const int64_t gy = cdiv(g.M, TL::BM), gx = cdiv(g.N, TL::BN);
  if (gy > 65535 || gx * gy * splits > 0x7fffffffLL || splits > 65535) return 0;
  hipLaunchKernelGGL((gemm_bf16_kernel<TL, ACT_NONE, false, float>), dim3((unsigned)gx, (unsigned)gy, (unsigned)splits),
                     dim3(TL::THREADS), 0, stream, g);
  CORTEX_CHECK_LAUNCH("gemm_bf16_kernel (K split)");
  return 1;
}

int launch_res_dw(const GemmArgs& g, hipStream_t stream) { return launch_res_dw_impl(g, stream); }

int try_gemm_bf16(const GemmArgs& g, int x_dtype, int w_dtype, int w_layout, int compute, hipStream_t stream) {
  if (compute != DT_BF16 || w_layout != 0 || x_dtype != DT_BF16 || (w_dtype != DT_BF16 && w_dtype != DT_I8)) return 0;
  if (g.norm != NORM_NONE || g.K % 64 != 0 || g.N % 8 != 0 || g.M <= 0 || g.N <= 0) return 0;
  if (g.M > 0x7fffffff || g.N > 0x7fffffff || g.K > 0x7fffffff) return 0;
  const bool w8 = w_dtype == DT_I8;
  if (!aligned16(g.x) || (g.ld_x * 2) % 16 || !aligned16(g.w) || (g.ld_w * (w8 ? 1 : 2)) % 16) return 0;
  if (g.w_scale && !aligned16(g.w_scale)) return 0;
  if (g.bias && (g.bias_dtype != DT_F32 || !aligned16(g.bias))) return 0;
  const bool res = g.res != nullptr;
  if (res && (g.res_dtype != DT_F32 || g.out_dtype != DT_F32 || !aligned16(g.res) || g.ld_res % 8)) return 0;
  const bool out_bf16 = g.out_dtype == DT_BF16;
  if (!out_bf16 && g.out_dtype != DT_F32) return 0;
  if (!aligned16(g.out) || g.ld_out % 8) return 0;
  // Residual (fp32 in/out) GEMMs are memory bound.  While 128 x 128 tiles give at most one
  // workgroup per CU: those tiles with K split over two wave groups (eight wavefronts per CU).
  // Larger grids (B >= 64 in the forward, the activation rows no longer in the infinity
  // cache): 256 x 128 tiles with a three-stage ring (144 KiB), whose extra stage of lead covers
  // the longer load latency and whose taller tile halves the weight refill per row.  Measured
  // forward at B = 64 / 128 / 256: 1.467 / 2.816 / 5.93 ms with the K-split tiles, 1.393 /
  // 2.647 / 5.42 ms with these.
  if (res) {
    if (g.act || g.K % 128) return 0;
    if (!w8 && g.N % 128 == 0 && cdiv(g.M, 128) * cdiv(g.N, 128) > cu_count())
      return launch<B256x128s3, ACT_NONE, true, float, bf16, bf16>(g, stream);
    return w8 ? launch<B128x128s2k2w, ACT_NONE, true, float, bf16, int8_t>(g, stream)
              : launch<B128x128s2k2, ACT_NONE, true, float, bf16, bf16>(g, stream);
  }
  if (w8) {
    if (out_bf16)
      return g.act ? dispatch<ACT_GELU, false, bf16, int8_t>(g, stream)
                   : dispatch<ACT_NONE, false, bf16, int8_t>(g, stream);
    return g.act ? dispatch<ACT_GELU, false, float, int8_t>(g, stream)
                 : dispatch<ACT_NONE, false, float, int8_t>(g, stream);
  }
  if (out_bf16)
    return g.act ? dispatch<ACT_GELU, false, bf16>(g, stream) : dispatch<ACT_NONE, false, bf16>(g, stream);
  return g.act ? dispatch<ACT_GELU, false, float>(g, stream) : dispatch<ACT_NONE, false, float>(g, stream);
}

}  // namespace cortex

using namespace cortex;

extern "C" int cortex_linear_w8a8(int64_t M, int64_t N, int64_t K, const int8_t* x, int64_t ld_x, float a_scale,
                                  const int8_t* w, int64_t ld_w, const float* w_scale, const float* bias, int act,
                                  const float* res, int64_t ld_res, int64_t res_rows, void* out, int out_dtype,
                                  float out_scale, int64_t ld_out, hipStream_t stream) {
  const char* who = "cortex_linear_w8a8";
  CORTEX_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: need M >= 0, N > 0, K > 0", who);
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= 0x7fffffffLL, "%s: size too large", who);
  CORTEX_CHECK_ARG(K % 128 == 0 && N % 8 == 0, "%s: K must be a multiple of 128 and N of 8", who);
  CORTEX_CHECK_ARG(act == ACT_NONE || act == ACT_GELU, "%s: act must be 0 (none) or 1 (GELU)", who);
  CORTEX_CHECK_ARG(out_dtype == DT_F32 || out_dtype == DT_I8, "%s: out must be fp32 or int8", who);
  CORTEX_CHECK_ARG(!(res && (out_dtype != DT_F32 || act != ACT_NONE)), "%s: a residual needs fp32 out and no act", who);
  CORTEX_CHECK_ARG(x && w && out && a_scale > 0.0f && (out_dtype == DT_F32 || out_scale > 0.0f),
                   "%s: null pointer or non-positive scale", who);
  CORTEX_CHECK_ARG(res_rows >= 0 && ld_x >= K && ld_w >= K && ld_out >= N && (!res || ld_res >= N),
                   "%s: row strides too small", who);
  CORTEX_CHECK_ARG(aligned16(x) && aligned16(w) && ld_x % 16 == 0 && ld_w % 16 == 0 && aligned16(out) &&
                       ld_out % 8 == 0 && (!w_scale || aligned16(w_scale)) && (!bias || aligned16(bias)) &&
                       (!res || (aligned16(res) && ld_res % 4 == 0)),
                   "%s: operands must be 16-byte aligned rows", who);
  GemmArgs g = {};
  g.M = M;
  g.N = N;
  g.K = K;
  g.x = x;
  g.ld_x = ld_x;
  g.w = w;
  g.ld_w = ld_w;
  g.w_scale = w_scale;
  g.bias = bias;
  g.bias_dtype = DT_F32;
  g.act = act;
  g.res = res;
  g.res_dtype = DT_F32;
  g.ld_res = ld_res;
  g.res_rows = res_rows;
  g.out = out;
  g.out_dtype = out_dtype;
  g.ld_out = ld_out;
  g.vec = 1;
  g.a_scale = a_scale;
  g.out_inv_scale = out_dtype == DT_I8 ? 1.0f / out_scale : 0.0f;
  const int ncu = cu_count();
  const int64_t t128 = cdiv(M, 128) * cdiv(N, 128), t256 = cdiv(M, 256) * cdiv(N, 256);
  int st;
  if (out_dtype == DT_I8) {
    const bool wide = N % 256 == 0 && t256 >= ncu * 15 / 16;
    if (act == ACT_GELU)
      st = wide ? launch<B256x256s2, ACT_GELU, false, int8_t, int8_t>(g, stream)
                : launch<B128x128s2, ACT_GELU, false, int8_t, int8_t>(g, stream);
    else
      st = wide ? launch<B256x256s2, ACT_NONE, false, int8_t, int8_t>(g, stream)
                : launch<B128x128s2, ACT_NONE, false, int8_t, int8_t>(g, stream);
  } else if (res) {
    st = (K % 256 == 0 && t128 <= ncu) ? launch<B128x128s2k2, ACT_NONE, true, float, int8_t>(g, stream)
                                       : launch<B128x128s2, ACT_NONE, true, float, int8_t>(g, stream);
  } else {
    st = act == ACT_GELU ? launch<B128x128s2, ACT_GELU, false, float, int8_t>(g, stream)
                         : launch<B128x128s2, ACT_NONE, false, float, int8_t>(g, stream);
  }
  if (st < 0) return st;
  if (st == 0) {
    set_error("%s: grid too large", who);
    return E_INVALID;
  }
  return OK;
}

extern "C" int cortex_norm_linear_fused(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, int norm,
                                        const void* gamma, const void* beta, int gamma_dtype, float eps, int w_dtype,
                                        const void* w, int64_t ld_w, const float* w_scale, const float* bias, int act,
                                        int out_dtype, void* out, int64_t ld_out, hipStream_t stream) {
  const char* who = "cortex_norm_linear_fused";
  CORTEX_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: need M >= 0, N > 0, K > 0", who);
  if (M == 0) return OK;
  CORTEX_CHECK_ARG(M <= 0x7fffffffLL && N <= 0x7fffffffLL, "%s: size too large", who);
  CORTEX_CHECK_ARG(K % 64 == 0 && K <= 512 && N % 8 == 0, "%s: need K a multiple of 64 up to 512 and N of 8", who);
  CORTEX_CHECK_ARG(norm == NORM_RMS || norm == NORM_LAYER, "%s: norm must be 1 (layer) or 2 (rms)", who);
  CORTEX_CHECK_ARG((gamma || norm == NORM_RMS) && (gamma_dtype == DT_F32 || gamma_dtype == DT_BF16),
                   "%s: gamma must be fp32 or bf16 (NULL only with RMS)", who);
  CORTEX_CHECK_ARG(w_dtype == DT_BF16 || w_dtype == DT_I8, "%s: weight must be bf16 or int8", who);
  CORTEX_CHECK_ARG(act == ACT_NONE || act == ACT_GELU, "%s: act must be 0 (none) or 1 (GELU)", who);
  CORTEX_CHECK_ARG(out_dtype == DT_BF16 || out_dtype == DT_F32, "%s: out must be bf16 or fp32", who);
  CORTEX_CHECK_ARG(x && w && out && eps >= 0.0f, "%s: null pointer or negative eps", who);
  CORTEX_CHECK_ARG(ld_x >= K && ld_w >= K && ld_out >= N, "%s: row strides too small", who);
  CORTEX_CHECK_ARG(aligned16(x) && ld_x % 8 == 0 && aligned16(w) && ld_w % (w_dtype == DT_I8 ? 16 : 8) == 0 &&
                       aligned16(out) && ld_out % 8 == 0 && (!w_scale || aligned16(w_scale)) &&
                       (!bias || aligned16(bias)) && (!gamma || aligned16(gamma)) && (!beta || aligned16(beta)),
                   "%s: operands must be 16-byte aligned rows", who);
  CORTEX_CHECK_ARG(N * ld_w * (w_dtype == DT_I8 ? 1 : 2) < (1LL << 31), "%s: weight larger than 2 GiB", who);
  NormGemmArgs a{M, N, K, reinterpret_cast<const bf16*>(x), ld_x, norm, gamma, norm == NORM_LAYER ? beta : nullptr,
                 gamma_dtype, eps, w, ld_w, w_scale, bias, out, ld_out, 1};
  int st;
  const bool gelu = act == ACT_GELU, obf = out_dtype == DT_BF16;
  if (norm == NORM_RMS && !gamma && w_dtype == DT_BF16 && M * ld_x * 2 < (1LL << 32)) {
    // rows as given and 1 / rms on the accumulator: the tiled GEMM sums the squares itself
    GemmArgs g = {};
    g.M = M;
    g.N = N;
    g.K = K;
    g.x = x;
    g.ld_x = ld_x;
    g.w = w;
    g.ld_w = ld_w;
    g.w_scale = w_scale;
    g.bias = bias;
    g.bias_dtype = DT_F32;
    g.act = act;
    g.out = out;
    g.out_dtype = out_dtype;
    g.ld_out = ld_out;
    g.vec = 1;
    g.rms_eps = eps;
    st = obf ? (gelu ? dispatch_rs<ACT_GELU, bf16>(g, stream) : dispatch_rs<ACT_NONE, bf16>(g, stream))
             : (gelu ? dispatch_rs<ACT_GELU, float>(g, stream) : dispatch_rs<ACT_NONE, float>(g, stream));
  } else if (w_dtype == DT_I8) {
    st = obf ? (gelu ? dispatch_norm<int8_t, ACT_GELU, bf16>(a, stream) : dispatch_norm<int8_t, ACT_NONE, bf16>(a, stream))
             : (gelu ? dispatch_norm<int8_t, ACT_GELU, float>(a, stream) : dispatch_norm<int8_t, ACT_NONE, float>(a, stream));
  } else {
    st = obf ? (gelu ? dispatch_norm<bf16, ACT_GELU, bf16>(a, stream) : dispatch_norm<bf16, ACT_NONE, bf16>(a, stream))
             : (gelu ? dispatch_norm<bf16, ACT_GELU, float>(a, stream) : dispatch_norm<bf16, ACT_NONE, float>(a, stream));
  }
  if (st < 0) return st;
  if (st == 0) {
    set_error("%s: grid too large", who);
    return E_INVALID;
  }
  return OK;
}
