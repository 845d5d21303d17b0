// Arguments shared by the general and the fast attention kernels.
#pragma once

#include "common.h"

namespace cortex {

struct AttnArgs {
  int64_t B, H, Lq, Lk, Dh;
  const void* q;
  int64_t q_sb, q_sh, q_sl;
  const void* k;
  int64_t k_sb, k_sh, k_sl;
  const void* v;
  int64_t v_sb, v_sh, v_sl;
  const int64_t* kv_off;  // (B+1) CSR row offsets (row index scaled by k_sl / v_sl)
  const int64_t* kv_len;  // (B,) valid keys per sample
  const uint8_t* key_mask;
  int64_t km_sb;
  const uint8_t* block_mask;
  int64_t bm_sb, n_qt, n_kt, block_l, block_e;
  float scale_log2;
  void* out;
  int64_t o_sb, o_sh, o_sl;
  int vec;
};

// bf16, head dim 64, no per-key or block mask, 16-byte aligned rows
// (attention_fast.hip).  Returns 1 when it launched, 0 when the request is outside
// its specialisation (the caller then runs the general kernel), negative on error.
int try_attention_fast(const AttnArgs& a, int dtype, hipStream_t stream);

}  // namespace cortex
