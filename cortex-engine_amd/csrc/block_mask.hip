// Temporal tile mask on the device (reference cortex/kernels/sparse_xattn.py:152-200).
//
// Latent i sits at time centre float32(i) / L * T (IEEE single, left to right).  Query
// tile qi spans [int(first centre) - w, int(last centre) + w] (int() truncates; the
// centres increase with i, so the tile's min and max are its first and last centre).
// Key tile kj of a sample spans [min t, max t] over its events; the pair is allowed
// iff the two intervals overlap.  A key tile with no event of the sample (past the
// sample's end in a per-sample CSR layout) is not allowed.
//
// One wavefront per key tile: the min/max reduction over its events, then the
// interval test against every query tile.  Integer work; bit-exact.
#include <hip/hip_runtime.h>

#include "common.h"

namespace cortex {

namespace {

struct TmArgs {
  const int64_t* t;
  int64_t t_stride, E;
  const int64_t* off;  // (B+1) CSR offsets, or null: one sample of E events
  int64_t n_latents, max_time_bins, window, block_l, block_e, n_q, n_k;
  uint8_t* out;
  int64_t out_sb;
};

__global__ __launch_bounds__(256) void temporal_mask_kernel(TmArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t kj = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (kj >= a.n_k) return;  // wave-uniform
  int64_t s0 = 0, s1 = a.E;
  if (a.off) {
    s0 = a.off[b];
    s1 = a.off[b + 1];
  }
  const int64_t e0 = s0 + kj * a.block_e;
  const int64_t e1 = min(e0 + a.block_e, s1);
  uint8_t* out = a.out + b * a.out_sb + kj;
  if (e0 >= e1) {  // no event of this sample in the tile
    for (int64_t qi = lane; qi < a.n_q; qi += 64) out[qi * a.n_k] = 0;
    return;
  }
  int64_t tmin = INT64_MAX, tmax = INT64_MIN;
  for (int64_t e = e0 + lane; e < e1; e += 64) {
    const int64_t v = a.t[e * a.t_stride];
    tmin = min(tmin, v);
    tmax = max(tmax, v);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    tmin = min(tmin, (int64_t)__shfl_xor((long long)tmin, m, 64));
    tmax = max(tmax, (int64_t)__shfl_xor((long long)tmax, m, 64));
  }
  const float L = (float)a.n_latents, T = (float)a.max_time_bins;
  for (int64_t qi = lane; qi < a.n_q; qi += 64) {
    const int64_t first = qi * a.block_l;
    const int64_t last = min(first + a.block_l - 1, a.n_latents - 1);
    const float c_lo = __fmul_rn(__fdiv_rn((float)first, L), T);
    const float c_hi = __fmul_rn(__fdiv_rn((float)last, L), T);
    const int64_t lo = (int64_t)c_lo - a.window;  // centres >= 0: the cast truncates like int()
    const int64_t hi = (int64_t)c_hi + a.window;
    out[qi * a.n_k] = (tmin <= hi && tmax >= lo) ? 1 : 0;
  }
}

}  // namespace

}  // namespace cortex

using namespace cortex;

extern "C" int cortex_temporal_block_mask(const int64_t* event_times, int64_t t_stride, int64_t E,
                                          const int64_t* offsets, int64_t B, int64_t n_latents,
                                          int64_t max_time_bins, int64_t window_bins, int64_t block_l,
                                          int64_t block_e, int64_t n_q, int64_t n_k, uint8_t* out, int64_t out_sb,
                                          hipStream_t stream) {
  CORTEX_CHECK_ARG(E >= 0 && B >= 0 && n_q >= 0 && n_k >= 0, "cortex_temporal_block_mask: negative size");
  CORTEX_CHECK_ARG(n_latents > 0 && n_latents <= (1 << 24) && max_time_bins >= 0,
                   "cortex_temporal_block_mask: n_latents must be in [1, 2^24] and max_time_bins >= 0");
  CORTEX_CHECK_ARG(block_l > 0 && block_e > 0, "cortex_temporal_block_mask: tile sizes must be positive");
  CORTEX_CHECK_ARG(offsets != nullptr || B == 1, "cortex_temporal_block_mask: B > 1 needs CSR offsets");
  if (B == 0 || n_q == 0 || n_k == 0) return OK;
  CORTEX_CHECK_ARG(out != nullptr && (E == 0 || event_times != nullptr), "cortex_temporal_block_mask: null pointer");
  CORTEX_CHECK_ARG(B <= 65535, "cortex_temporal_block_mask: B %lld > 65535", (long long)B);
  CORTEX_CHECK_ARG(cdiv(n_k, (int64_t)4) <= 0x7fffffffLL, "cortex_temporal_block_mask: too many key tiles");
  TmArgs a{event_times, t_stride, E, offsets, n_latents, max_time_bins, window_bins, block_l, block_e, n_q, n_k,
           out, out_sb};
  hipLaunchKernelGGL(temporal_mask_kernel, dim3((unsigned)cdiv(n_k, (int64_t)4), (unsigned)B), dim3(256), 0, stream,
                     a);
  CORTEX_CHECK_LAUNCH("temporal_mask_kernel");
  return OK;
}
