// Shared device/host helpers for the Cortex gfx950 kernels.
//
// Conventions used by every kernel in this library:
//  * one 64-lane wavefront is the unit of cooperation (CDNA4);
//  * MFMA fragments are 8 consecutive K-elements per lane: lane l owns row/column
//    (l % 16) and the K slice [8*(l/16), 8*(l/16)+8) of a 16 x 32 operand block;
//    bf16 feeds one v_mfma_f32_16x16x32_bf16, fp32 feeds eight
//    v_mfma_f32_16x16x4_f32 (slot j of every lane forms the j-th 16x16x4 step,
//    i.e. the K order is permuted identically on both operands);
//  * the 16x16 fp32 accumulator holds element (4*(l/16)+i, l%16) in register i.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

namespace cortex {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// dtype codes shared with include/cortex_hip.h; DT_BF16_FRAG is a weight layout code, not a
// tensor dtype: bf16 weights in MFMA fragment order (cortex_frag_weight)
enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_I8 = 3, DT_I32 = 4, DT_I64 = 5, DT_U8 = 6, DT_BF16_FRAG = 7 };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(int8_t x) { return (float)(int)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }

template <class T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }  // RNE
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }  // RNE

// Fragment of 8 K-consecutive operand values for one lane.
template <class T>
struct Frag;
template <>
struct Frag<bf16> {
  bf16x8 v;
};
template <>
struct Frag<float> {
  f32x8 v;
};

// acc(16x16, fp32) += A(16 x 32) * B(32 x 16) with both operands as fragments.
__device__ __forceinline__ void mfma_16x16x32(f32x4& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mfma_16x16x32(f32x4& acc, const Frag<float>& a, const Frag<float>& b) {
#pragma unroll
  for (int j = 0; j < 8; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[j], b.v[j], acc, 0, 0, 0);
}

// Output stores written through the L2 to memory at device scope (SC1).  A kernel's outputs
// are read by the next kernel, mostly on other XCDs; written through as they are produced,
// they leave no dirty lines behind for the L2 write-back at the end of the kernel, which
// otherwise starts only after the last store.  (Non-temporal stores skip that write-back too
// but also bypass the infinity cache that the next kernel reads from.)
//
// The stores are the compiler's own buffer stores with the SC1 cache-policy bit, so it counts
// them in its vmcnt waits and inserts the wait states their data registers need.  WtOut holds
// the buffer descriptor of one output tensor (built once per kernel from its base, which must
// be uniform: a kernel argument); a store passes its 32-bit byte offset from that base.  A
// tensor of 4 GiB or more is written with plain stores.  No code may read the stored bytes back
// in the same kernel.
constexpr int CPOL_SC1 = 16;  // cache-policy operand: SC1 (device scope)
struct WtOut {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t base_lo;
  bool wt;
  // raw buffer (stride 0) over 4 GiB; word 3: the 32-bit data format that untyped accesses need
  __device__ __forceinline__ WtOut(const void* base, int64_t bytes, bool wt_)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000)),
        base_lo((uint32_t)(uintptr_t)base),
        wt(wt_ && bytes < (1ll << 32)) {}
  template <class V>
  __device__ __forceinline__ void operator()(V* p, const V& v) const {
    if (!wt) {
      *p = v;
      return;
    }
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    const uint32_t off = (uint32_t)(uintptr_t)p - base_lo;  // the byte offset (below 4 GiB)
    if constexpr (sizeof(V) == 16) {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rsrc, off, 0, CPOL_SC1);
    } else if constexpr (sizeof(V) == 8) {
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, v), rsrc, off, 0, CPOL_SC1);
    } else {
      static_assert(sizeof(V) == 4, "4-, 8- or 16-byte stores");
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), rsrc, off, 0, CPOL_SC1);
    }
  }
};

// When write-through pays (measured on the Cortex-S forward, B = 32 / 64 / 256):
//  * a GEMM or attention launch whose grid is a single wave of one workgroup per CU (MI355X:
//    256 CUs) produces all its outputs at the end, so their write-back would run after the
//    last store: written through, MLP-up, MLP-down and the kv projection are 1.8-2.5 us faster
//    at B = 32.  With more workgroups than CUs the early ones' lines are written back while
//    later ones run, and writing through only adds partial-line writes (3-12 % slower);
//  * the LayerNorm row pass gains at every size (a streaming kernel with bf16 output);
//  * the tokenizer gains while its output stays small (16 MiB at B = 32; 33 MiB at B = 64 loses).
constexpr int WT_MAX_WORKGROUPS = 256;
constexpr int64_t WT_MAX_BYTES = 24ll << 20;
__device__ __forceinline__ bool wt_one_wave() {
  return (int64_t)gridDim.x * gridDim.y * gridDim.z <= WT_MAX_WORKGROUPS;
}
__device__ __forceinline__ bool wt_fits(int64_t bytes) { return bytes <= WT_MAX_BYTES; }

// Operand element type of the direct-to-LDS GEMM loops: a 16-byte fragment per lane and the
// MFMA that consumes it (bf16: 8 K-elements, fp32 accumulators; int8: 16 K-elements, int32
// accumulators).  Both read 16 bytes per lane per operand, so LDS layouts carry over.
template <class TIN>
struct Operand;
template <>
struct Operand<bf16> {
  typedef bf16x8 frag;
  typedef f32x4 accum;
  typedef float elem;
  static constexpr int EPC = 8;  // elements per 16-byte chunk
  static __device__ __forceinline__ accum mma(const frag& w, const frag& a, const accum& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, a, c, 0, 0, 0);
  }
};
template <>
struct Operand<int8_t> {
  typedef i32x4 frag;
  typedef i32x4 accum;
  typedef int elem;
  static constexpr int EPC = 16;
  static __device__ __forceinline__ accum mma(const frag& w, const frag& a, const accum& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(w, a, c, 0, 0, 0);
  }
};

// Exact int8 -> bf16 widening of 8 values (every int8 value is a bf16 value); the
// compiler emits one sign-extending byte convert per value and one pack per pair.
__device__ __forceinline__ bf16x8 widen_i8x8(uint2 raw) {
  const int8_t* p = reinterpret_cast<const int8_t*>(&raw);
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (bf16)(float)(int)p[j];
  return v;
}

// Widening rider of a launch: up to WR_MAX int8 arrays widened exactly to bf16
// (dst[i][e] = src[i][e]) by `blocks` extra workgroups of the launch's grid, each taking
// `chunk` consecutive elements of the concatenated arrays (WR_CHUNK, or WR_CHUNK_SMALL for a
// launch whose own workgroups leave most CUs idle, so that the rider spreads over all of them).
// The row kernels are HBM-bound streams with idle issue slots, so a few MB of weights ride along
// for about their transfer time and no launch of their own.  Element counts are multiples of 16
// and both arrays 16-byte aligned; the bf16 rows are written through (read by later kernels).
constexpr int WR_MAX = 8;
constexpr int64_t WR_CHUNK = 32768, WR_CHUNK_SMALL = 8192;
struct WidenRider {
  const int8_t* src[WR_MAX];
  bf16* dst[WR_MAX];
  int64_t end[WR_MAX];  // cumulative element counts
  int fk[WR_MAX];       // log2 of the row length K: dst in MFMA fragment order (cortex_frag_weight); 0: as src
  int count;
  int blocks;           // rider workgroups (0: none)
  int64_t chunk;        // elements per rider workgroup
};
// One whole chunk with every load in flight before the stores (256 threads, U loads each).
template <int U, class Put>
__device__ __forceinline__ void widen_chunk(const int8_t* src, const Put& put) {
  i32x4 raw[U];
#pragma unroll
  for (int u = 0; u < U; ++u) raw[u] = *reinterpret_cast<const i32x4*>(src + (u * 256 + threadIdx.x) * 16);
#pragma unroll
  for (int u = 0; u < U; ++u) put((u * 256 + threadIdx.x) * 16, raw[u]);
}
__device__ __forceinline__ void widen_rider_run(const WidenRider& r, int blk) {
  const int64_t lo = (int64_t)blk * r.chunk, hi = lo + r.chunk;
  int64_t s0 = 0;
  for (int s = 0; s < r.count; ++s) {
    const int64_t s1 = r.end[s], a = lo > s0 ? lo : s0, b = hi < s1 ? hi : s1;
    if (a < b) {
      const WtOut store(r.dst[s], (s1 - s0) * 2, true);
      const int8_t* src = r.src[s] + (a - s0);
      bf16* dst = r.dst[s] + (a - s0);
      const int fk = r.fk[s];
      if (fk != 0) {
        // fragment-order destination (cortex_frag_weight's layout): the 16-element units are
        // taken tile by tile, 64 consecutive units = one 16-row x 64-K tile (unit l of a tile: row
        // l % 16, K 16 (l / 16) .. +15), so a wavefront reads 16 rows x 64 bytes and writes two
        // whole 1 KiB blocks (block (n / 16) * (K / 32) + k / 32, lane n % 16 + 16 ((k / 8) % 4))
        const int tk = fk - 6;  // log2 of the 64-K tiles per 16-row band
        for (int64_t i = threadIdx.x * 16; i < b - a; i += (int64_t)blockDim.x * 16) {
          const int64_t u = (a - s0 + i) >> 4, w = u >> 6;
          const int l = (int)(u & 63);
          const int64_t n = ((w >> tk) << 4) + (l & 15), k = ((w & ((1ll << tk) - 1)) << 6) + ((l >> 4) << 4);
          const i32x4 raw = *reinterpret_cast<const i32x4*>(r.src[s] + (n << fk) + k);
          const int64_t off = ((((n >> 4) << (fk - 5)) + (k >> 5)) << 9) + ((((k >> 3) & 3) << 4) + (n & 15)) * 8;
          store(reinterpret_cast<bf16x8*>(r.dst[s] + off), widen_i8x8(make_uint2((uint32_t)raw[0], (uint32_t)raw[1])));
          store(reinterpret_cast<bf16x8*>(r.dst[s] + off + 128),
                widen_i8x8(make_uint2((uint32_t)raw[2], (uint32_t)raw[3])));
        }
        s0 = s1;
        continue;
      }
      auto put = [&](int64_t i, const i32x4& raw) {
        store(reinterpret_cast<bf16x8*>(dst + i), widen_i8x8(make_uint2((uint32_t)raw[0], (uint32_t)raw[1])));
        store(reinterpret_cast<bf16x8*>(dst + i + 8), widen_i8x8(make_uint2((uint32_t)raw[2], (uint32_t)raw[3])));
      };
      if (b - a == WR_CHUNK && blockDim.x == 256) {
        widen_chunk<(int)(WR_CHUNK / (256 * 16))>(src, put);
      } else if (b - a == WR_CHUNK_SMALL && blockDim.x == 256) {
        widen_chunk<(int)(WR_CHUNK_SMALL / (256 * 16))>(src, put);
      } else {
        for (int64_t i = threadIdx.x * 16; i < b - a; i += (int64_t)blockDim.x * 16)
          put(i, *reinterpret_cast<const i32x4*>(src + i));
      }
    }
    s0 = s1;
  }
}
// The rider re-cut into workgroups of `chunk` elements.
inline void rider_chunk(WidenRider& r, int64_t chunk) {
  const int64_t total = r.count ? r.end[r.count - 1] : 0;
  r.chunk = chunk;
  r.blocks = (int)((total + chunk - 1) / chunk);
}

// A value every lane of the wavefront holds alike (a row index, a loaded table index), moved to
// scalar registers: the compiler cannot prove such values uniform, and would otherwise keep
// their 64-bit address arithmetic in vector registers (quarter-rate multiplies per lane).
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Cross-lane reductions inside one wavefront.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, in every lane: DPP adds inside each 16-lane row (quad xor 1,
// quad xor 2, row rotate 4, row rotate 8), then the four row sums read out as scalars.
// A few cycles per step instead of an LDS round trip per shuffle (wave_sum).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x124>(v);
  v += dpp_mov<0x128>(v);
  const int iv = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48)));
}

// Workgroups go to the 8 XCDs round-robin by linear id (id % 8).  A kernel whose
// neighbouring work items share operands (the column tiles of one row panel, the
// query blocks or heads of one sample) indexes them by xcd_affine(id, total): XCD x
// then takes the x-th contiguous eighth, and the shared operands are fetched into
// one XCD's L2 instead of eight.  (A bijection on [0, total); identity unless 8 | total.)
__device__ __forceinline__ int xcd_affine(int id, int total) {
  return (total & 7) ? id : (id & 7) * (total >> 3) + (id >> 3);
}

// One LayerNorm pass over the EPL values a lane holds of one row spread over a wavefront:
// element (j / 4) * 256 + 4 lane + j % 4 in v[j]; two passes (mean, then squared deviations).
template <int EPL>
__device__ __forceinline__ void ln_regs(float (&v)[EPL], float inv_k, float eps, const float* __restrict__ gamma,
                                        const float* __restrict__ beta, int lane) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) s += v[j];
  const float mean = wave_sum(s) * inv_k;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const float d = v[j] - mean;
    ss += d * d;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) * inv_k + eps);
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    // element k = (j / 4) * 256 + lane * 4 + (j % 4)
    const int k = (j >> 2) * 256 + lane * 4;
    const float4 gm = gamma ? *reinterpret_cast<const float4*>(gamma + k) : make_float4(1.f, 1.f, 1.f, 1.f);
    const float4 bt = beta ? *reinterpret_cast<const float4*>(beta + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    v[j] = (v[j] - mean) * rstd * gm.x + bt.x;
    v[j + 1] = (v[j + 1] - mean) * rstd * gm.y + bt.y;
    v[j + 2] = (v[j + 2] - mean) * rstd * gm.z + bt.z;
    v[j + 3] = (v[j + 3] - mean) * rstd * gm.w + bt.w;
  }
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// erf-form GELU, as torch.nn.GELU() with approximate='none': 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }

// Same GELU for results that are rounded to bf16 (relative step 2^-8).  With
// a = |x| and Q(a) = erfc(a / sqrt 2) / 2 the standard normal upper tail, both signs
// reduce to
//   GELU(x) = max(x, 0) - a Q(a)      (x >= 0: x (1 - Q); x < 0: x Q)
// log2 Q(a) is smooth on [0, 6]; the degree-6 polynomial below is a weighted
// least-squares (near-minimax) fit of it with |error| <= 6.5e-5 there, so Q and the
// result carry a relative error <= 5e-5 (0.012 bf16 steps).  Past a = 6 the clamped
// term 6 Q(6) < 6e-9 stands in for a Q(a) (absolute error < 6e-9), and x = +inf
// gives +inf.  Cost: 9 VALU operations and one exp2 per element.
__device__ __forceinline__ float gelu_erf_bf16out(float x) {
  const float a = fminf(fabsf(x), 6.0f);
  float p = 2.299003427e-05f;
  p = fmaf(p, a, -6.110987160e-04f);
  p = fmaf(p, a, 7.195549086e-03f);
  p = fmaf(p, a, -5.118525401e-02f);
  p = fmaf(p, a, -4.612721205e-01f);
  p = fmaf(p, a, -1.150174141e+00f);
  p = fmaf(p, a, -1.000064850e+00f);
  return fmaf(-a, __builtin_amdgcn_exp2f(p), fmaxf(x, 0.0f));
}

}  // namespace cortex

// ----------------------------------------------------------------------------
// Host-side error plumbing for the C ABI: every entry point returns 0 or a
// negative status and records a message retrievable by cortex_last_error().
// ----------------------------------------------------------------------------
namespace cortex {
enum Status : int {
  OK = 0,
  E_INVALID = -1,      // bad shape / dtype / stride / pointer
  E_UNSUPPORTED = -2,  // valid request this build does not implement
  E_LAUNCH = -3,       // HIP launch or runtime error
  E_WORKSPACE = -4,    // workspace too small
};
void set_error(const char* fmt, ...);
// Widening riders (rowops.hip): build one from the C-ABI arrays (0 or a negative status), and
// launch one on a grid of its own.
struct WidenRider;
int make_rider(const char* who, int n, const void* const* src, void* const* dst, const int64_t* count,
               const int64_t* frag_k, WidenRider* r);
int widen_launch(const WidenRider& wr, hipStream_t stream);
}  // namespace cortex

#define CORTEX_CHECK_ARG(cond, ...)          \
  do {                                       \
    if (!(cond)) {                           \
      ::cortex::set_error(__VA_ARGS__);      \
      return ::cortex::E_INVALID;            \
    }                                        \
  } while (0)

#define CORTEX_CHECK_LAUNCH(what)                                                   \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess) {                                                         \
      ::cortex::set_error("%s: launch failed: %s", what, hipGetErrorString(_e));    \
      return ::cortex::E_LAUNCH;                                                    \
    }                                                                               \
  } while (0)
