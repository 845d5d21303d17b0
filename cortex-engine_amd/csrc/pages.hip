// Window assembly from device-resident event pages (the streaming cache's gather), and
// the batched page write that fills them.
//
// A streaming server keeps each session's spike events in pages of consecutive time
// bins, stored once on the device with ABSOLUTE bin numbers.  A decode window is the
// concatenation of its pages in bin order; its model input needs bins relative to
// the window start.  One workgroup per (page -> window rows) item copies the page's
// neuron ids and values and rewrites its bins as bin - shift, straight into the
// forward's input buffer.  Pure copies: bit-exact, HBM bound (48 B per event).
#include <hip/hip_runtime.h>

#include "common.h"

namespace cortex {

namespace {

struct GatherArgs {
  const int64_t* pool;  // (num_pages, 3, page_events): neuron id, absolute bin, value
  int64_t num_pages, page_events;
  const int64_t* plan;  // (n_items, 4): page id, event count, first output row, bin shift
  int64_t n_items;
  int64_t* out;  // field f of row r at out[f * field_stride + r]
  int64_t field_stride, out_rows;
  int32_t* err;
};

__global__ __launch_bounds__(256) void gather_pages_kernel(GatherArgs a) {
  const int64_t item = blockIdx.x;
  const int64_t* p = a.plan + item * 4;
  const int64_t page = p[0], n = p[1], dst = p[2], shift = p[3];
  if (page < 0 || page >= a.num_pages || n < 0 || n > a.page_events || dst < 0 || dst > a.out_rows - n) {
    if (threadIdx.x == 0 && a.err) atomicOr(a.err, 4);  // malformed item: nothing written
    return;
  }
  const int64_t* src = a.pool + page * 3 * a.page_events;
  for (int64_t e = threadIdx.x; e < n; e += blockDim.x) {
    a.out[dst + e] = src[e];
    a.out[a.field_stride + dst + e] = src[a.page_events + e] - shift;
    a.out[2 * a.field_stride + dst + e] = src[2 * a.page_events + e];
  }
}

struct ScatterArgs {
  const int64_t* src;  // field f of staged event r at src[f * field_stride + r]
  int64_t field_stride, src_rows;
  const int64_t* plan;  // (n_items, 3): page id, event count, first staged row
  int64_t n_items;
  int64_t* pool;
  int64_t num_pages, page_events;
  int32_t* err;
};

__global__ __launch_bounds__(256) void scatter_pages_kernel(ScatterArgs a) {
  const int64_t* p = a.plan + (int64_t)blockIdx.x * 3;
  const int64_t page = p[0], n = p[1], s0 = p[2];
  if (page < 0 || page >= a.num_pages || n < 0 || n > a.page_events || s0 < 0 || s0 > a.src_rows - n) {
    if (threadIdx.x == 0 && a.err) atomicOr(a.err, 4);
    return;
  }
  int64_t* dst = a.pool + page * 3 * a.page_events;
  for (int64_t e = threadIdx.x; e < n; e += blockDim.x) {
    dst[e] = a.src[s0 + e];
    dst[a.page_events + e] = a.src[a.field_stride + s0 + e];
    dst[2 * a.page_events + e] = a.src[2 * a.field_stride + s0 + e];
  }
}

}  // namespace

}  // namespace cortex

using namespace cortex;

extern "C" int cortex_scatter_event_pages(const int64_t* src, int64_t field_stride, int64_t src_rows,
                                          const int64_t* plan, int64_t n_items, int64_t* pool, int64_t num_pages,
                                          int64_t page_events, int32_t* err, hipStream_t stream) {
  CORTEX_CHECK_ARG(num_pages >= 0 && page_events >= 0 && n_items >= 0 && src_rows >= 0,
                   "cortex_scatter_event_pages: negative size");
  if (n_items == 0) return OK;
  CORTEX_CHECK_ARG(src && plan && pool, "cortex_scatter_event_pages: null pointer");
  CORTEX_CHECK_ARG(field_stride >= src_rows, "cortex_scatter_event_pages: field_stride < src_rows");
  CORTEX_CHECK_ARG(n_items <= 0x7fffffffLL, "cortex_scatter_event_pages: too many items");
  ScatterArgs a{src, field_stride, src_rows, plan, n_items, pool, num_pages, page_events, err};
  hipLaunchKernelGGL(scatter_pages_kernel, dim3((unsigned)n_items), dim3(256), 0, stream, a);
  CORTEX_CHECK_LAUNCH("scatter_pages_kernel");
  return OK;
}

extern "C" int cortex_gather_event_pages(const int64_t* pool, int64_t num_pages, int64_t page_events,
                                         const int64_t* plan, int64_t n_items, int64_t* out, int64_t field_stride,
                                         int64_t out_rows, int32_t* err, hipStream_t stream) {
  CORTEX_CHECK_ARG(num_pages >= 0 && page_events >= 0 && n_items >= 0 && out_rows >= 0,
                   "cortex_gather_event_pages: negative size");
  if (n_items == 0) return OK;
  CORTEX_CHECK_ARG(pool && plan && out, "cortex_gather_event_pages: null pointer");
  CORTEX_CHECK_ARG(field_stride >= out_rows, "cortex_gather_event_pages: field_stride < out_rows");
  CORTEX_CHECK_ARG(n_items <= 0x7fffffffLL, "cortex_gather_event_pages: too many items");
  GatherArgs a{pool, num_pages, page_events, plan, n_items, out, field_stride, out_rows, err};
  hipLaunchKernelGGL(gather_pages_kernel, dim3((unsigned)n_items), dim3(256), 0, stream, a);
  CORTEX_CHECK_LAUNCH("gather_pages_kernel");
  return OK;
}
