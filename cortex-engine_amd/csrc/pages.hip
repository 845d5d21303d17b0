// Window assembly from device-resident event pages (the streaming cache's gather).
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

}  // namespace

}  // namespace cortex

using namespace cortex;

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
