// Spike tokenizer and ragged-event pack for gfx950.
//
//   * pack plan: a device-side stable counting sort of the events by batch index
//     (no host synchronisation): per-chunk histograms, one scan over (chunk,
//     sample), then in-order ranking inside each chunk -- one launch for small
//     plans, three for large ones.
//     It yields CSR offsets (B+1), the CSR row of every event and the source
//     event of every CSR row -- exactly the stable argsort + exclusive cumsum of
//     the reference pack (cortex/models/cortex.py:140-160).
//   * row writer: one wavefront per output row, 16-byte coalesced stores, that
//     either gathers the three embedding rows and adds them
//     ((N[nid] + T[tb]) + V[val], reference cortex/kernels/tokenizer.py:81) or
//     copies an existing token row.  Output rows are CSR order (E rows) or the
//     padded (B, E_max) layout with its bool mask (cortex.py:146-147,163-164).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "common.h"

namespace cortex {

// Error-flag bits (device int32, OR-ed).
constexpr int ERR_TOKEN_INDEX = 1;  // neuron/time/value index outside its table
constexpr int ERR_BATCH_INDEX = 2;  // batch index outside [0, B)
constexpr int PACK_FLAG_CLEAR_ERR = 1;  // cortex_pack_plan flags: zero err_flag before the plan

constexpr int PACK_MAX_B = 8192;   // LDS histogram bins per chunk
constexpr int PACK_MAX_CHUNKS = 1024;

__host__ __device__ inline int64_t pack_chunk_size(int64_t E) {
  int64_t c = 1024;
  int64_t need = cdiv(E, PACK_MAX_CHUNKS);
  if (need > c) c = cdiv(need, 64) * 64;
  return c;
}

// Lanes of the wavefront whose sample index equals this lane's, among the lanes with
// `valid` set (0 <= b < 2^bits).  One test covers the common case of a single sample;
// otherwise one ballot per bit of b, so the cost does not grow with the number of
// distinct samples the 64 events hold (up to 64 for shuffled events).
__device__ __forceinline__ uint64_t same_sample_lanes(int b, bool valid, int bits) {
  uint64_t same = __ballot(valid);
  if (same == 0) return 0ull;
  // sorted batches: the 64 events usually belong to one sample
  const int b0 = __builtin_amdgcn_readlane(b, __ffsll((unsigned long long)same) - 1);
  if (__ballot(valid && b == b0) == same) return valid ? same : 0ull;
  for (int k = 0; k < bits; ++k) {
    const bool bit = (b >> k) & 1;
    const uint64_t m = __ballot(bit);
    same &= bit ? m : ~m;
  }
  return valid ? same : 0ull;
}

// Clears the error word before any later atomic of this kernel or of the next ones ORs into
// it: an atomic exchange whose result is consumed, so that the wave waits for it.
__device__ __forceinline__ void clear_err_word(int32_t* err, int* sink) {
  const int old = __hip_atomic_exchange(err, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old == 0x7fffffff) *sink = 0;  // never true for the flag bits: keeps the exchange's wait
}

// Bits of a sample index below B.
__host__ __device__ inline int sample_bits(int B) {
  int bits = 0;
  while ((1 << bits) < B) ++bits;
  return bits;
}

// Small fills (kept as kernels so that callers may capture them in a graph).
__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Whether every range of the wide sorted check (pack_sorted_kernel's status words: 1 sorted
// and in range, 2 not) was sorted; the whole workgroup takes part and gets the same answer.
// A null status list means no check ran.
__device__ bool ranges_sorted(const int* __restrict__ status, int n_status, int* s_flag) {
  if (!status) return false;
  if (threadIdx.x == 0) *s_flag = 1;
  __syncthreads();
  for (int i = threadIdx.x; i < n_status; i += blockDim.x)
    if (status[i] != 1) *s_flag = 0;
  __syncthreads();
  return *s_flag != 0;
}

// The three launches below return at once when the wide sorted check found every range
// sorted (the identity plan it wrote is the plan).

// 1) per-chunk histogram of batch indices.
__global__ __launch_bounds__(256) void pack_count_kernel(const int64_t* __restrict__ bidx, int64_t s_bidx, int64_t E,
                                                          int B, int64_t C, int* __restrict__ counts,
                                                          int* __restrict__ err, const int* __restrict__ status,
                                                          int n_status) {
  __shared__ int hist[PACK_MAX_B];
  __shared__ int sorted_flag;
  if (ranges_sorted(status, n_status, &sorted_flag)) return;
  const int chunk = blockIdx.x;
  for (int b = threadIdx.x; b < B; b += blockDim.x) hist[b] = 0;
  __syncthreads();
  const int64_t beg = (int64_t)chunk * C;
  const int64_t end = min(E, beg + C);
  bool bad = false;
  const int lane = threadIdx.x & 63, bits = sample_bits(B);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t i0 = beg; i0 < end; i0 += blockDim.x) {  // every lane runs the same trip count
    const int64_t i = i0 + threadIdx.x;
    int64_t b = -1;
    if (i < end) {
      b = bidx[i * s_bidx];
      if (b < 0 || b >= B) {
        bad = true;
        b = -1;
      }
    }
    // one atomic per distinct sample among the wave's 64 events, by its lowest lane
    // (sorted batches would otherwise send 64 atomics to one LDS word)
    const uint64_t same = same_sample_lanes((int)b, b >= 0, bits);
    if (b >= 0 && (same & lt_mask) == 0) atomicAdd(&hist[b], (int)__popcll(same));
  }
  if (bad && err) atomicOr(err, ERR_BATCH_INDEX);
  __syncthreads();
  for (int b = threadIdx.x; b < B; b += blockDim.x) counts[(int64_t)chunk * B + b] = hist[b];
}

// 2) exclusive scan over chunks per sample (in place), then over samples.
__global__ __launch_bounds__(1024) void pack_scan_kernel(int* __restrict__ counts, int nchunks, int B,
                                                          int64_t* __restrict__ offsets, int32_t* __restrict__ ident,
                                                          const int* __restrict__ status, int n_status) {
  __shared__ int64_t part[1024];
  __shared__ int totals[PACK_MAX_B];
  __shared__ int sorted_flag;
  const int tid = threadIdx.x;
  if (ranges_sorted(status, n_status, &sorted_flag)) {
    if (ident && tid == 0) *ident = 1;
    return;
  }
  for (int b = tid; b < B; b += blockDim.x) {
    int run = 0;
    for (int c = 0; c < nchunks; ++c) {
      int t = counts[(int64_t)c * B + b];
      counts[(int64_t)c * B + b] = run;
      run += t;
    }
    totals[b] = run;
  }
  __syncthreads();
  // each thread owns a contiguous span of samples
  const int per = (B + blockDim.x - 1) / blockDim.x;
  const int b0 = tid * per;
  int64_t local = 0;
  for (int b = b0; b < min(B, b0 + per); ++b) local += totals[b];
  part[tid] = local;
  __syncthreads();
  // Hillis-Steele inclusive scan of the 1024 partials
  for (int off = 1; off < (int)blockDim.x; off <<= 1) {
    int64_t v = (tid >= off) ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int64_t run = part[tid] - local;  // exclusive prefix of this span
  for (int b = b0; b < min(B, b0 + per); ++b) {
    offsets[b] = run;
    run += totals[b];
  }
  if (tid == blockDim.x - 1) offsets[B] = part[tid];
  if (ident && tid == 0) *ident = 0;  // this plan always writes `order`
}

// 3) in-order ranking inside each chunk: one wavefront walks its chunk 64 events
//    at a time; lanes holding the same sample are ranked by lane order.
__global__ __launch_bounds__(64) void pack_rank_kernel(const int64_t* __restrict__ bidx, int64_t s_bidx, int64_t E,
                                                        int B, int64_t C, const int* __restrict__ chunk_base,
                                                        const int64_t* __restrict__ offsets,
                                                        int64_t* __restrict__ order, int64_t* __restrict__ dst_rows,
                                                        int64_t* __restrict__ rank, const int* __restrict__ status,
                                                        int n_status) {
  __shared__ int64_t next[PACK_MAX_B];
  __shared__ int sorted_flag;
  if (ranges_sorted(status, n_status, &sorted_flag)) return;
  const int chunk = blockIdx.x;
  const int lane = threadIdx.x;
  for (int b = lane; b < B; b += 64) next[b] = offsets[b] + chunk_base[(int64_t)chunk * B + b];
  __syncthreads();
  const int64_t beg = (int64_t)chunk * C;
  const int64_t end = min(E, beg + C);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int bits = sample_bits(B);
  for (int64_t base = beg; base < end; base += 64) {
    const int64_t i = base + lane;
    int64_t b = -1;
    if (i < end) {
      b = bidx[i * s_bidx];
      if (b < 0 || b >= B) b = -1;  // counted as an error by pack_count_kernel
    }
    const uint64_t same = same_sample_lanes((int)b, b >= 0, bits);
    int64_t row0 = 0;
    if (b >= 0) {
      row0 = next[b];  // every lane of a sample reads the same word ...
      const int64_t row = row0 + __popcll(same & lt_mask);
      order[row] = i;
      if (dst_rows) dst_rows[i] = row;
      if (rank) rank[i] = row - offsets[b];
    }
    __syncthreads();  // single wavefront: the reads above complete before the update
    if (b >= 0 && (same & lt_mask) == 0) next[b] = row0 + __popcll(same);  // ... and its lowest lane advances it
    __syncthreads();
  }
}

// Small plans (B <= 1024, E <= 65536) in ONE launch: one workgroup of 16 waves, wave w
// owning the contiguous event chunk w.  Per-wave histograms in LDS, the two scans
// (over waves per sample, then over samples), then the same in-order ranking as
// pack_rank_kernel.  Same results as the three-launch path, a third of its launches.
// Without ranks, sorted indices are recognised first and take the identity plan.  When the
// caller asks for an identity flag, a sorted plan sets it and leaves `order` unwritten (a
// consumer then maps row r to event r); an unsorted one clears it and writes `order`.
constexpr int PS_WAVES = 16;
constexpr int PS_MAX_B = 1024;
constexpr int64_t PS_MAX_E = 65536;
constexpr int PS_UNROLL = 16;

// Sorted batch indices (the collate order) need no sort: the plan is the identity and
// offsets[s] is the first event of sample s.  Event e (index b, the event before it bp; -1
// for the first event) writes its identity row and the offsets of the samples bp+1 .. b
// (empty ones too), which start at e; the last event closes the samples after it.  Returns
// false, writing nothing, when e breaks the order or an index is out of range.  (bp is -1
// only for the first event: a negative index before e is out of range, and taking it as the
// loop start would write offsets[] below index 0.)
__device__ __forceinline__ bool sorted_event(int64_t e, int64_t b, int64_t bp, int64_t E, int B,
                                             int64_t* __restrict__ offsets, int64_t* __restrict__ order,
                                             int64_t* __restrict__ dst_rows) {
  if (b < 0 || b >= B || bp > b || (e > 0 && bp < 0)) return false;
  if (order) order[e] = e;
  if (dst_rows) dst_rows[e] = e;
  for (int64_t s = bp + 1; s <= b; ++s) offsets[s] = e;
  if (e == E - 1)
    for (int64_t s = b + 1; s <= B; ++s) offsets[s] = E;
  return true;
}

// The batch index of the event before this lane's: the previous lane's value (lane 0 loads
// its own).  `b` is this lane's index, `e` its event; only lanes with 0 < e < E use the result,
// and lane 0 loads only then (every lane takes part in the shuffle).
__device__ __forceinline__ int64_t prev_index(int64_t b, int64_t e, int64_t E, const int64_t* __restrict__ bidx,
                                              int64_t s_bidx, int lane) {
  const int64_t up = __shfl_up(b, 1, 64);
  if (lane != 0) return up;
  return (e > 0 && e < E) ? bidx[(e - 1) * s_bidx] : -1;
}

// Above PS_ONE_E events the sorted check runs wide first: one workgroup per PS_SORTED_EV
// events (one per thread) applies sorted_event to its range and records in
// status[blockIdx.x] whether the range (with the event before it) was sorted and in range: 1
// yes, 2 no.  pack_small_kernel then returns at once when every status is 1 and otherwise
// recomputes the whole plan.  Up to PS_ONE_E events pack_small_kernel makes the check itself
// (one round of loads per thread), so a plan is one launch; above that one workgroup is
// latency-bound (9.5 us at 16384 events against about 2 + 1.5 us for the wide check and the
// status read).
constexpr int PS_SORTED_EV = 256;
constexpr int PS_ONE_UNROLL = 4;
constexpr int64_t PS_ONE_E = 64 * PS_WAVES * PS_ONE_UNROLL;

__global__ __launch_bounds__(PS_SORTED_EV) void pack_sorted_kernel(const int64_t* __restrict__ bidx, int64_t s_bidx,
                                                                   int64_t E, int B, int64_t* __restrict__ offsets,
                                                                   int64_t* __restrict__ order,
                                                                   int64_t* __restrict__ dst_rows,
                                                                   int* __restrict__ status, int32_t* clear_err,
                                                                   WidenRider wr) {
  // the plan's workgroups first; a widening rider's after them, on the CUs the plan leaves idle
  const int nplan = (int)gridDim.x - wr.blocks;
  if ((int)blockIdx.x >= nplan) {
    widen_rider_run(wr, (int)blockIdx.x - nplan);
    return;
  }
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  if (clear_err && blockIdx.x == 0 && threadIdx.x == 0) clear_err_word(clear_err, &bad);
  __syncthreads();
  const int64_t e = (int64_t)blockIdx.x * PS_SORTED_EV + threadIdx.x;
  const int64_t b = e < E ? bidx[e * s_bidx] : 0;
  const int64_t bp = prev_index(b, e, E, bidx, s_bidx, threadIdx.x & 63);
  if (e < E && !sorted_event(e, b, bp, E, B, offsets, order, dst_rows)) bad = 1;
  __syncthreads();
  if (threadIdx.x == 0) status[blockIdx.x] = bad ? 2 : 1;
}

__global__ __launch_bounds__(1024) void pack_small_kernel(const int64_t* __restrict__ bidx, int64_t s_bidx, int64_t E,
                                                          int B, int64_t* __restrict__ offsets,
                                                          int64_t* __restrict__ order, int64_t* __restrict__ dst_rows,
                                                          int64_t* __restrict__ rank, int32_t* __restrict__ err,
                                                          const int* __restrict__ status, int n_status,
                                                          bool try_sorted, int32_t* __restrict__ ident,
                                                          bool clear_err, WidenRider wr) {
  if (blockIdx.x > 0) {  // workgroup 0 is the plan; any others carry a widening rider
    widen_rider_run(wr, (int)blockIdx.x - 1);
    return;
  }
  __shared__ int cnt[PS_WAVES * PS_MAX_B];  // per-wave counts, then per-wave next CSR row
  __shared__ int first[PS_MAX_B];           // CSR offset of each sample
  __shared__ int wsum[PS_WAVES];
  __shared__ int unsorted;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // (every OR into err below follows at least one barrier)
  if (clear_err && err && tid == 0) clear_err_word(err, &wsum[0]);
  if (status) {  // after pack_sorted_kernel: nothing left to do when every range was sorted
    if (tid == 0) unsorted = 0;
    __syncthreads();
    for (int i = tid; i < n_status; i += blockDim.x)
      if (status[i] != 1) unsorted = 1;
    __syncthreads();
    if (!unsorted) {
      if (ident && tid == 0) *ident = 1;
      return;
    }
  } else if (try_sorted) {  // E <= PS_ONE_E: the sorted check here, every load issued first
    if (tid == 0) unsorted = 0;
    __syncthreads();
    int64_t bv[PS_ONE_UNROLL];
#pragma unroll
    for (int u = 0; u < PS_ONE_UNROLL; ++u) {
      const int64_t e = (int64_t)u * blockDim.x + tid;
      bv[u] = e < E ? bidx[e * s_bidx] : 0;
    }
    bool my_bad = false;
    int64_t* const ord = ident ? nullptr : order;  // with the flag, a sorted plan writes no order
#pragma unroll
    for (int u = 0; u < PS_ONE_UNROLL; ++u) {
      const int64_t e = (int64_t)u * blockDim.x + tid;
      const int64_t bp = prev_index(bv[u], e, E, bidx, s_bidx, lane);
      if (e < E && !sorted_event(e, bv[u], bp, E, B, offsets, ord, dst_rows)) my_bad = true;
    }
    if (my_bad) unsorted = 1;
    // the identity writes complete before the full plan below rewrites every offset and
    // every CSR row of `order`
    __threadfence_block();
    __syncthreads();
    if (!unsorted) {
      if (ident && tid == 0) *ident = 1;
      return;
    }
  }
  if (ident && tid == 0) *ident = 0;
  for (int i = tid; i < PS_WAVES * B; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  const int64_t C = cdiv(E, (int64_t)PS_WAVES);
  const int64_t beg = w * C, end = min(E, beg + C);
  int* mine = cnt + w * B;
  const int bits = sample_bits(B);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  bool bad = false;
  for (int64_t base = beg; base < end; base += 64 * PS_UNROLL) {  // PS_UNROLL loads in flight per lane
    int64_t bv[PS_UNROLL];
#pragma unroll
    for (int u = 0; u < PS_UNROLL; ++u) {
      const int64_t i = base + 64 * u + lane;
      bv[u] = i < end ? bidx[i * s_bidx] : (int64_t)B;
    }
#pragma unroll
    for (int u = 0; u < PS_UNROLL; ++u) {
      int64_t b = bv[u];
      if (base + 64 * u + lane < end && (b < 0 || b >= B)) bad = true;
      if (b < 0 || b >= B) b = -1;
      // one update per distinct sample in the 64 events, by its lowest lane (distinct
      // samples: distinct words of this wave's own row of cnt)
      const uint64_t same = same_sample_lanes((int)b, b >= 0, bits);
      if (b >= 0 && (same & lt_mask) == 0) mine[b] += __popcll(same);
    }
  }
  if (bad && err) atomicOr(err, ERR_BATCH_INDEX);
  __syncthreads();
  // per sample: exclusive prefix over the waves (in place) and the sample's total
  int total_b = 0;
  if (tid < B) {
    for (int ww = 0; ww < PS_WAVES; ++ww) {
      const int t = cnt[ww * B + tid];
      cnt[ww * B + tid] = total_b;
      total_b += t;
    }
  }
  // exclusive scan of the totals over samples: lane scan, then over the 16 wave sums
  int incl = total_b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int wbase = 0;
  for (int ww = 0; ww < w; ++ww) wbase += wsum[ww];
  if (tid < B) {
    const int excl = wbase + incl - total_b;
    first[tid] = excl;
    offsets[tid] = excl;
  }
  if (tid == 0) {
    int all = 0;
    for (int ww = 0; ww < PS_WAVES; ++ww) all += wsum[ww];
    offsets[B] = all;
  }
  __syncthreads();
  for (int i = tid; i < PS_WAVES * B; i += blockDim.x) cnt[i] += first[i % B];
  __syncthreads();
  // in-order ranking inside the chunk; only this wave touches its row of `cnt`
  for (int64_t base = beg; base < end; base += 64 * PS_UNROLL) {
    int64_t bv[PS_UNROLL];
#pragma unroll
    for (int u = 0; u < PS_UNROLL; ++u) {
      const int64_t i = base + 64 * u + lane;
      bv[u] = i < end ? bidx[i * s_bidx] : -1;
    }
#pragma unroll
    for (int u = 0; u < PS_UNROLL; ++u) {
      const int64_t i = base + 64 * u + lane;
      const int64_t b = (bv[u] < 0 || bv[u] >= B) ? -1 : bv[u];
      const uint64_t same = same_sample_lanes((int)b, b >= 0, bits);
      if (b >= 0) {
        // all lanes of a sample read its word before its lowest lane advances it (one
        // wavefront's LDS operations complete in program order)
        const int row0 = mine[b];
        const int64_t row = row0 + __popcll(same & lt_mask);
        order[row] = i;
        if (dst_rows) dst_rows[i] = row;
        if (rank) rank[i] = row - first[b];
        if ((same & lt_mask) == 0) mine[b] = row0 + __popcll(same);
      }
    }
  }
}

// Row writer -------------------------------------------------------------------

template <class T>
__device__ __forceinline__ T add_rn(T a, T b) {
  return from_f32<T>(to_f32(a) + to_f32(b));
}
template <>
__device__ __forceinline__ float add_rn<float>(float a, float b) {
  return a + b;
}

// 16-byte vector of T
template <class T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  T v[N];
};

struct RowArgs {
  // sources
  const void* tab[3];      // neuron, time, value tables (table mode)
  int64_t tab_rows[3];
  int64_t tab_ld[3];
  const int64_t* ids[3];   // per-event indices (table mode)
  int64_t ids_stride[3];
  const void* src;         // (E, D) token rows (copy mode)
  int64_t src_ld;
  // mapping
  int64_t E;               // number of events
  int64_t D;
  const int64_t* order;    // CSR row -> source event (nullable: identity)
  const int32_t* ident;    // nullable: when *ident != 0 the plan is the identity and order is unused
  const int64_t* offsets;  // padded mode: (B+1) CSR offsets
  const int64_t* csr_end;  // CSR mode (nullable): number of valid CSR rows (offsets[B])
  int64_t B, E_max;        // padded mode
  // output
  void* out;
  int64_t out_ld;
  uint8_t* mask;           // padded mode (B, E_max), nullable
  int* err;
};

// MODE_TABLE: gather-add from three tables; MODE_COPY: copy src rows.
enum { MODE_TABLE = 0, MODE_COPY = 1 };

template <class T, int MODE, bool PADDED, bool VEC>
__global__ __launch_bounds__(256) void row_writer_kernel(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t rows = PADDED ? a.B * a.E_max : a.E;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (r >= rows) return;
  int64_t e;
  if (PADDED) {
    const int64_t b = r / a.E_max, j = r - b * a.E_max;
    const int64_t o0 = a.offsets[b], cnt = a.offsets[b + 1] - o0;
    const bool identity = !a.order || (a.ident && *a.ident);
    e = (j < cnt) ? (identity ? o0 + j : a.order[o0 + j]) : -1;
    if (a.mask && lane == 0) a.mask[r] = (j < cnt) ? 1 : 0;
  } else {
    // rows past offsets[B] exist only when some batch indices were invalid: zero them
    const bool identity = !a.order || (a.ident && *a.ident);
    e = (a.csr_end && r >= *a.csr_end) ? -1 : (identity ? r : a.order[r]);
  }
  if (e >= a.E) e = -1;  // defensive: never follow a corrupt order entry
  T* out = reinterpret_cast<T*>(a.out) + r * a.out_ld;
  const WtOut store(a.out, rows * a.out_ld * (int64_t)sizeof(T), wt_fits(rows * a.D * (int64_t)sizeof(T)));
  const T* s0 = nullptr;
  const T* s1 = nullptr;
  const T* s2 = nullptr;
  if (e >= 0) {
    if (MODE == MODE_TABLE) {
      const int64_t i0 = a.ids[0][e * a.ids_stride[0]];
      const int64_t i1 = a.ids[1][e * a.ids_stride[1]];
      const int64_t i2 = a.ids[2][e * a.ids_stride[2]];
      if (i0 < 0 || i0 >= a.tab_rows[0] || i1 < 0 || i1 >= a.tab_rows[1] || i2 < 0 || i2 >= a.tab_rows[2]) {
        if (lane == 0 && a.err) atomicOr(a.err, ERR_TOKEN_INDEX);
        e = -1;  // never read out of bounds: the row is written as zeros
      } else {
        s0 = reinterpret_cast<const T*>(a.tab[0]) + i0 * a.tab_ld[0];
        s1 = reinterpret_cast<const T*>(a.tab[1]) + i1 * a.tab_ld[1];
        s2 = reinterpret_cast<const T*>(a.tab[2]) + i2 * a.tab_ld[2];
      }
    } else {
      s0 = reinterpret_cast<const T*>(a.src) + e * a.src_ld;
    }
  }
  if (VEC) {
    using V = Vec16<T>;
    constexpr int NV = V::N;
    for (int64_t d = (int64_t)lane * NV; d < a.D; d += 64 * NV) {
      V o;
      if (e < 0) {
#pragma unroll
        for (int q = 0; q < NV; ++q) o.v[q] = from_f32<T>(0.0f);
      } else if (MODE == MODE_TABLE) {
        const V x = *reinterpret_cast<const V*>(s0 + d);
        const V y = *reinterpret_cast<const V*>(s1 + d);
        const V z = *reinterpret_cast<const V*>(s2 + d);
#pragma unroll
        for (int q = 0; q < NV; ++q) o.v[q] = add_rn<T>(add_rn<T>(x.v[q], y.v[q]), z.v[q]);
      } else {
        o = *reinterpret_cast<const V*>(s0 + d);
      }
      store(reinterpret_cast<V*>(out + d), o);
    }
  } else {
    for (int64_t d = lane; d < a.D; d += 64) {
      T o;
      if (e < 0) {
        o = from_f32<T>(0.0f);
      } else if (MODE == MODE_TABLE) {
        o = add_rn<T>(add_rn<T>(s0[d], s1[d]), s2[d]);
      } else {
        o = s0[d];
      }
      out[d] = o;
    }
  }
}

// Tokens in CSR order from the tables (the API tokenizer's main case), TOK_ROWS rows per
// wavefront.  A row is a chain of dependent loads (order -> the three indices -> the three
// table rows), so every load of one link is issued for all rows before any is waited on; with
// the plan's identity flag set (sorted batch indices) the first link is r itself.  Rows past
// *csr_end and rows with an index outside its table are zero (the latter set the error bit).
// 16-byte aligned rows, D a multiple of the 16-byte vector.
constexpr int TOK_ROWS = 4;

template <class T>
__global__ __launch_bounds__(256) void tokenize_csr_kernel(RowArgs a) {
  constexpr int R = TOK_ROWS;
  using V = Vec16<T>;
  constexpr int NV = V::N;
  const int lane = threadIdx.x & 63;
  // the wavefront's rows, their events and table indices are alike in every lane: scalar
  // registers and scalar address arithmetic
  const int64_t r0 = ((int64_t)blockIdx.x * (blockDim.x >> 6) + wave_uniform((int)threadIdx.x >> 6)) * R;
  if (r0 >= a.E) return;
  const bool identity = !a.order || (a.ident && *a.ident);
  const int64_t end = a.csr_end ? *a.csr_end : a.E;
  int64_t e[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i;
    e[i] = (r < a.E && r < end) ? (identity ? r : a.order[r]) : -1;
    if (e[i] >= a.E) e[i] = -1;  // defensive: never follow a corrupt order entry
    e[i] = wave_uniform(e[i]);
  }
  int64_t id[R][3];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int t = 0; t < 3; ++t) id[i][t] = e[i] >= 0 ? wave_uniform(a.ids[t][e[i] * a.ids_stride[t]]) : 0;
  const T* src[R][3];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (e[i] >= 0 && (id[i][0] < 0 || id[i][0] >= a.tab_rows[0] || id[i][1] < 0 || id[i][1] >= a.tab_rows[1] ||
                      id[i][2] < 0 || id[i][2] >= a.tab_rows[2])) {
      if (lane == 0 && a.err) atomicOr(a.err, ERR_TOKEN_INDEX);
      e[i] = -1;  // never read out of bounds: the row is written as zeros
    }
#pragma unroll
    for (int t = 0; t < 3; ++t) src[i][t] = reinterpret_cast<const T*>(a.tab[t]) + (e[i] >= 0 ? id[i][t] : 0) * a.tab_ld[t];
  }
  const WtOut store(a.out, a.E * a.out_ld * (int64_t)sizeof(T), wt_fits(a.E * a.D * (int64_t)sizeof(T)));
  for (int64_t d = (int64_t)lane * NV; d < a.D; d += 64 * NV) {
    V x[R][3];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int t = 0; t < 3; ++t)
        if (e[i] >= 0) x[i][t] = *reinterpret_cast<const V*>(src[i][t] + d);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (r0 + i >= a.E) break;
      V o;
#pragma unroll
      for (int q = 0; q < NV; ++q)
        o.v[q] = e[i] >= 0 ? add_rn<T>(add_rn<T>(x[i][0].v[q], x[i][1].v[q]), x[i][2].v[q]) : from_f32<T>(0.0f);
      store(reinterpret_cast<V*>(reinterpret_cast<T*>(a.out) + (r0 + i) * a.out_ld + d), o);
    }
  }
}

}  // namespace cortex

using namespace cortex;

template <class T, int MODE>
static int launch_rows(const RowArgs& a, bool padded, hipStream_t stream) {
  const int64_t rows = padded ? a.B * a.E_max : a.E;
  if (rows == 0) return OK;
  const int waves_per_block = 4;
  if (cdiv(rows, waves_per_block) > 0x7fffffffLL) {
    set_error("cortex row writer: %lld rows exceed the grid limit", (long long)rows);
    return E_INVALID;
  }
  const dim3 grid((unsigned)cdiv(rows, waves_per_block));
  constexpr int NV = 16 / sizeof(T);
  bool vec = (a.D % NV == 0) && ((uintptr_t)a.out % 16 == 0) && ((a.out_ld * (int64_t)sizeof(T)) % 16 == 0);
  if (MODE == MODE_TABLE) {
    for (int t = 0; t < 3; ++t)
      vec = vec && ((uintptr_t)a.tab[t] % 16 == 0) && ((a.tab_ld[t] * (int64_t)sizeof(T)) % 16 == 0);
  } else {
    vec = vec && ((uintptr_t)a.src % 16 == 0) && ((a.src_ld * (int64_t)sizeof(T)) % 16 == 0);
  }
  if (MODE == MODE_TABLE && !padded && vec) {
    const dim3 g((unsigned)cdiv(cdiv(rows, TOK_ROWS), waves_per_block));
    hipLaunchKernelGGL((tokenize_csr_kernel<T>), g, dim3(256), 0, stream, a);
  } else if (padded) {
    if (vec)
      hipLaunchKernelGGL((row_writer_kernel<T, MODE, true, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((row_writer_kernel<T, MODE, true, false>), grid, dim3(256), 0, stream, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((row_writer_kernel<T, MODE, false, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((row_writer_kernel<T, MODE, false, false>), grid, dim3(256), 0, stream, a);
  }
  CORTEX_CHECK_LAUNCH("cortex row writer");
  return OK;
}

template <int MODE>
static int dispatch_rows(int dtype, const RowArgs& a, bool padded, hipStream_t stream) {
  switch (dtype) {
    case DT_F32:
      return launch_rows<float, MODE>(a, padded, stream);
    case DT_BF16:
      return launch_rows<bf16, MODE>(a, padded, stream);
    case DT_F16:
      return launch_rows<f16, MODE>(a, padded, stream);
    default:
      set_error("unsupported token dtype %d (expected f32, bf16 or f16)", dtype);
      return E_UNSUPPORTED;
  }
}

extern "C" {

int64_t cortex_pack_workspace_bytes(int64_t E, int64_t B) {
  if (E <= 0 || B <= 0) return 0;
  const int64_t C = pack_chunk_size(E);
  const int64_t nchunks = cdiv(E, C);
  // per-chunk counts (three-launch plan) and one status word per sorted-check workgroup
  const int64_t words = nchunks * B + cdiv(E, (int64_t)PS_SORTED_EV);
  return words * (int64_t)sizeof(int);
}

}  // extern "C"

// The plan itself, shared by cortex_pack_plan (caller's workspace) and
// cortex_pack_plan_noalloc (the library's static scratch).  Every workspace word a
// launch reads was written by an earlier launch of the same call, so nothing in it
// needs clearing between calls.
static int pack_plan_impl(const char* who, const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B,
                          int64_t* offsets, int64_t* order, int64_t* dst_rows, int64_t* rank, void* workspace,
                          int64_t workspace_bytes, int32_t* err_flag, int32_t* identity, int flags,
                          hipStream_t stream, const WidenRider& wr = WidenRider{}) {
  const bool clear = (flags & PACK_FLAG_CLEAR_ERR) && err_flag != nullptr;
  CORTEX_CHECK_ARG(E >= 0 && B >= 1, "%s: need E >= 0 and B >= 1 (got E=%lld B=%lld)", who, (long long)E,
                   (long long)B);
  CORTEX_CHECK_ARG(B <= PACK_MAX_B, "%s: B=%lld exceeds the supported maximum %d", who, (long long)B, PACK_MAX_B);
  CORTEX_CHECK_ARG(offsets != nullptr, "%s: offsets must not be null", who);
  if (E == 0) {
    hipLaunchKernelGGL(fill_i64_kernel, dim3((unsigned)cdiv(B + 1, 256)), dim3(256), 0, stream, offsets, B + 1,
                       (int64_t)0);
    CORTEX_CHECK_LAUNCH("cortex_pack_plan(E=0)");
    if (clear) {
      hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, stream, err_flag, (int64_t)1, 0);
      CORTEX_CHECK_LAUNCH("cortex_pack_plan(E=0)");
    }
    if (identity) {  // the empty plan is the identity
      hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, stream, identity, (int64_t)1, 1);
      CORTEX_CHECK_LAUNCH("cortex_pack_plan(E=0)");
    }
    return widen_launch(wr, stream);
  }
  CORTEX_CHECK_ARG(batch_indices && order, "%s: batch_indices and order must not be null", who);
  const int64_t need = cortex_pack_workspace_bytes(E, B);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) {
    set_error("%s: workspace of %lld bytes is smaller than the required %lld", who, (long long)workspace_bytes,
              (long long)need);
    return E_WORKSPACE;
  }
  if (B <= PS_MAX_B && E <= PS_MAX_E) {
    // without ranks, the identity plan of sorted indices first: inside the one launch up to
    // PS_ONE_E events, above that in the wide pack_sorted_kernel (one status word per 1024
    // events, in the workspace: cortex_pack_workspace_bytes covers them)
    int* status = nullptr;
    const int n_status = (int)cdiv(E, (int64_t)PS_SORTED_EV);
    const bool one = rank == nullptr && E <= PS_ONE_E;
    // a widening rider joins the plan's first launch
    if (rank == nullptr && !one && workspace != nullptr && workspace_bytes >= n_status * (int64_t)sizeof(int)) {
      status = reinterpret_cast<int*>(workspace);
      hipLaunchKernelGGL(pack_sorted_kernel, dim3((unsigned)(n_status + wr.blocks)), dim3(PS_SORTED_EV), 0, stream,
                         batch_indices, s_bidx, E, (int)B, offsets, identity ? nullptr : order, dst_rows, status,
                         clear ? err_flag : nullptr, wr);
      CORTEX_CHECK_LAUNCH("pack_sorted_kernel");
    }
    const WidenRider& wr_small = status ? WidenRider{} : wr;
    hipLaunchKernelGGL(pack_small_kernel, dim3((unsigned)(1 + wr_small.blocks)), dim3(64 * PS_WAVES), 0, stream,
                       batch_indices, s_bidx, E, (int)B, offsets, order, dst_rows, rank, err_flag, status, n_status,
                       one, identity, clear && status == nullptr, wr_small);
    CORTEX_CHECK_LAUNCH("pack_small_kernel");
    return OK;
  }
  const int64_t C = pack_chunk_size(E);
  const int nchunks = (int)cdiv(E, C);
  int* counts = reinterpret_cast<int*>(workspace);
  // Without ranks, sorted indices first (the wide check, its status words after the counts):
  // the three launches then return at once.  The check also clears the error word.
  int* status = nullptr;
  const int n_status = (int)cdiv(E, (int64_t)PS_SORTED_EV);
  if (rank == nullptr) {
    status = counts + (int64_t)nchunks * B;
    hipLaunchKernelGGL(pack_sorted_kernel, dim3((unsigned)(n_status + wr.blocks)), dim3(PS_SORTED_EV), 0, stream,
                       batch_indices, s_bidx, E, (int)B, offsets, identity ? nullptr : order, dst_rows, status,
                       clear ? err_flag : nullptr, wr);
    CORTEX_CHECK_LAUNCH("pack_sorted_kernel");
  } else {
    if (clear) {
      hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, stream, err_flag, (int64_t)1, 0);
      CORTEX_CHECK_LAUNCH("cortex_pack_plan(clear)");
    }
    const int st = widen_launch(wr, stream);
    if (st != OK) return st;
  }
  hipLaunchKernelGGL(pack_count_kernel, dim3(nchunks), dim3(256), 0, stream, batch_indices, s_bidx, E, (int)B, C,
                     counts, err_flag, status, n_status);
  CORTEX_CHECK_LAUNCH("pack_count_kernel");
  hipLaunchKernelGGL(pack_scan_kernel, dim3(1), dim3(1024), 0, stream, counts, nchunks, (int)B, offsets, identity,
                     status, n_status);
  CORTEX_CHECK_LAUNCH("pack_scan_kernel");
  hipLaunchKernelGGL(pack_rank_kernel, dim3(nchunks), dim3(64), 0, stream, batch_indices, s_bidx, E, (int)B, C,
                     counts, offsets, order, dst_rows, rank, status, n_status);
  CORTEX_CHECK_LAUNCH("pack_rank_kernel");
  return OK;
}

// Scratch of cortex_pack_plan_noalloc: the per-chunk counts (three-launch plan) or the
// per-range status words (wide sorted check) that cortex_pack_plan keeps in the caller's
// workspace.  One copy per GPU, held until the process ends.  In host code `scratch`
// only names the symbol: its device address comes from hipGetSymbolAddress, once per
// device, and only that address is ever handed to a kernel.
constexpr int64_t PACK_SCRATCH_BYTES = (int64_t)4 << 20;
static __device__ __align__(256) int scratch[PACK_SCRATCH_BYTES / sizeof(int)];

constexpr int PACK_SCRATCH_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[PACK_SCRATCH_MAX_DEVICES];

// Device address of `scratch` on `dev`, looked up once per device with `dev` current.
static int pack_scratch_ptr(int dev, void** out) {
  if (dev < 0 || dev >= PACK_SCRATCH_MAX_DEVICES) {
    set_error("cortex_pack_plan_noalloc: device %d outside [0, %d)", dev, PACK_SCRATCH_MAX_DEVICES);
    return E_INVALID;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess || p == nullptr) {
      set_error("cortex_pack_plan_noalloc: scratch address on device %d: %s", dev,
                e != hipSuccess ? hipGetErrorString(e) : "null");
      return E_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return OK;
}

extern "C" {

int cortex_pack_plan(const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B, int64_t* offsets,
                     int64_t* order, int64_t* dst_rows, int64_t* rank, void* workspace, int64_t workspace_bytes,
                     int32_t* err_flag, int32_t* identity, int flags, hipStream_t stream) {
  return pack_plan_impl("cortex_pack_plan", batch_indices, s_bidx, E, B, offsets, order, dst_rows, rank, workspace,
                        workspace_bytes, err_flag, identity, flags, stream);
}

int cortex_pack_plan_widen(const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B, int64_t* offsets,
                           int64_t* order, int64_t* dst_rows, int64_t* rank, void* workspace,
                           int64_t workspace_bytes, int32_t* err_flag, int32_t* identity, int flags, int n_widen,
                           const void* const* widen_src, void* const* widen_dst, const int64_t* widen_count,
                           const int64_t* widen_frag_k, hipStream_t stream) {
  WidenRider wr;
  const int st = make_rider("cortex_pack_plan_widen", n_widen, widen_src, widen_dst, widen_count, widen_frag_k, &wr);
  if (st != OK) return st;
  rider_chunk(wr, WR_CHUNK_SMALL);  // the plan holds a few CUs: the rider takes all the others
  return pack_plan_impl("cortex_pack_plan_widen", batch_indices, s_bidx, E, B, offsets, order, dst_rows, rank,
                        workspace, workspace_bytes, err_flag, identity, flags, stream, wr);
}

int64_t cortex_pack_noalloc_max_workspace_bytes(void) { return PACK_SCRATCH_BYTES; }

int cortex_pack_plan_noalloc(const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B, int64_t* offsets,
                             int64_t* order, int64_t* dst_rows, int64_t* rank, int32_t* err_flag,
                             hipStream_t stream) {
  const int64_t need = cortex_pack_workspace_bytes(E, B);
  if (need > PACK_SCRATCH_BYTES) {
    set_error("cortex_pack_plan_noalloc: E=%lld, B=%lld needs %lld bytes of scratch, above its maximum of %lld "
              "(use cortex_pack_plan with a workspace)",
              (long long)E, (long long)B, (long long)need, (long long)PACK_SCRATCH_BYTES);
    return E_WORKSPACE;
  }
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("cortex_pack_plan_noalloc: device of the stream: %s", hipGetErrorString(e));
    return E_LAUNCH;
  }
  void* ws = nullptr;
  const int rc = pack_scratch_ptr(dev, &ws);
  if (rc != OK) return rc;
  return pack_plan_impl("cortex_pack_plan_noalloc", batch_indices, s_bidx, E, B, offsets, order, dst_rows, rank, ws,
                        PACK_SCRATCH_BYTES, err_flag, nullptr, 0, stream);
}

int cortex_tokenize(int dtype, int64_t D, const void* neuron_emb, int64_t n_neuron, int64_t ld_neuron,
                    const void* time_emb, int64_t n_time, int64_t ld_time, const void* value_emb, int64_t n_value,
                    int64_t ld_value, const int64_t* neuron_ids, int64_t s_nid, const int64_t* time_bins,
                    int64_t s_tb, const int64_t* values, int64_t s_val, int64_t E, const int64_t* order,
                    const int64_t* csr_end, const int64_t* offsets, int64_t B, int64_t E_max, void* out,
                    int64_t ld_out, uint8_t* mask, const int32_t* identity, int32_t* err_flag, hipStream_t stream) {
  CORTEX_CHECK_ARG(D > 0 && E >= 0, "cortex_tokenize: need D > 0 and E >= 0");
  CORTEX_CHECK_ARG(neuron_emb && time_emb && value_emb, "cortex_tokenize: null embedding table");
  CORTEX_CHECK_ARG(E == 0 || (neuron_ids && time_bins && values), "cortex_tokenize: null index array");
  CORTEX_CHECK_ARG(out != nullptr || (offsets ? B * E_max == 0 : E == 0), "cortex_tokenize: null output");
  CORTEX_CHECK_ARG(ld_out >= D && ld_neuron >= D && ld_time >= D && ld_value >= D,
                   "cortex_tokenize: row strides must be >= D");
  RowArgs a = {};
  a.tab[0] = neuron_emb;
  a.tab[1] = time_emb;
  a.tab[2] = value_emb;
  a.tab_rows[0] = n_neuron;
  a.tab_rows[1] = n_time;
  a.tab_rows[2] = n_value;
  a.tab_ld[0] = ld_neuron;
  a.tab_ld[1] = ld_time;
  a.tab_ld[2] = ld_value;
  a.ids[0] = neuron_ids;
  a.ids[1] = time_bins;
  a.ids[2] = values;
  a.ids_stride[0] = s_nid;
  a.ids_stride[1] = s_tb;
  a.ids_stride[2] = s_val;
  a.E = E;
  a.D = D;
  a.order = order;
  a.ident = identity;
  a.csr_end = csr_end;
  a.offsets = offsets;
  a.B = B;
  a.E_max = E_max;
  a.out = out;
  a.out_ld = ld_out;
  a.mask = mask;
  a.err = err_flag;
  const bool padded = offsets != nullptr;
  if (padded) CORTEX_CHECK_ARG(B >= 1 && E_max >= 0, "cortex_tokenize: padded output needs B >= 1, E_max >= 0");
  return dispatch_rows<MODE_TABLE>(dtype, a, padded, stream);
}

int cortex_pack_rows(int dtype, int64_t D, const void* src, int64_t ld_src, int64_t E, const int64_t* order,
                     const int64_t* csr_end, const int64_t* offsets, int64_t B, int64_t E_max, void* out,
                     int64_t ld_out, uint8_t* mask, hipStream_t stream) {
  CORTEX_CHECK_ARG(D > 0 && E >= 0, "cortex_pack_rows: need D > 0 and E >= 0");
  CORTEX_CHECK_ARG(E == 0 || src, "cortex_pack_rows: null source rows");
  CORTEX_CHECK_ARG(ld_out >= D && ld_src >= D, "cortex_pack_rows: row strides must be >= D");
  RowArgs a = {};
  a.src = src;
  a.src_ld = ld_src;
  a.E = E;
  a.D = D;
  a.order = order;
  a.csr_end = csr_end;
  a.offsets = offsets;
  a.B = B;
  a.E_max = E_max;
  a.out = out;
  a.out_ld = ld_out;
  a.mask = mask;
  const bool padded = offsets != nullptr;
  return dispatch_rows<MODE_COPY>(dtype, a, padded, stream);
}

}  // extern "C"
