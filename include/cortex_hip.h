/*
 * cortex_hip.h -- C ABI of libcortex_hip.so, the gfx950 (MI355X) kernels of the
 * Cortex-S inference forward.
 *
 * Conventions
 *   - Every entry point returns 0 on success or a negative status
 *     (-1 invalid argument, -2 unsupported combination, -3 launch error,
 *     -4 workspace too small); cortex_last_error() describes the last failure on
 *     the calling thread.  Nothing throws across the ABI.
 *   - All pointers are device pointers owned by the caller; the library keeps no
 *     pointer after returning.  Work is enqueued on `stream` (the caller's current
 *     stream) and the library never synchronises the host.
 *   - Shapes and strides are int64 element counts.  dtype codes:
 *     0 f32, 1 bf16, 2 f16, 3 int8, 4 int32, 5 int64, 6 uint8; weight code 7: a bf16
 *     weight in MFMA fragment order (cortex_frag_weight), where an entry point says so.
 *   - Index-range violations never read or write out of bounds: the offending row
 *     is written as zeros and a bit is OR-ed into the caller's device `err_flag`
 *     (1: token index outside its table, 2: batch index outside [0, B)).
 *
 * Reference interfaces (upstream repository, file:line) are cited per entry point.
 */
#ifndef CORTEX_HIP_H_
#define CORTEX_HIP_H_

#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version (1) and the last error message of the calling thread. */
int cortex_version(void);
const char* cortex_last_error(void);

/* ---- a2: stable pack of ragged events ------------------------------------
 * Replaces the bincount / stable argsort / exclusive cumsum of
 * _pack_events (cortex/models/cortex.py:140-160), without its two host syncs
 * (cortex.py:140,142): B is supplied by the caller.
 *   offsets  (B+1)  CSR offsets: sample b owns rows [offsets[b], offsets[b+1])
 *   order    (E)    source event of every CSR row (stable in event order)
 *   dst_rows (E)    CSR row of every event (nullable)
 *   rank     (E)    position of every event inside its sample (nullable)
 *   identity (1)    int32 (nullable): when given, a plan of sorted batch indices sets it
 *                   to 1 and leaves `order` unwritten (row r is event r); any other plan
 *                   sets it to 0 and writes `order`.  Consumers take the flag beside
 *                   `order` (cortex_tokenize, cortex_tokenize_ln).
 *   flags           CORTEX_PACK_CLEAR_ERR (1): set *err_flag to 0 before the plan ORs into
 *                   it, inside the plan's own first launch (a forward's error word starts
 *                   clean without a separate fill launch).
 * workspace: at least cortex_pack_workspace_bytes(E, B) bytes of device memory.
 * Sorted batch indices (the collate order) are recognised on the device when rank is
 * null: up to 4096 events the check and the plan are one launch; above (any E and B), the
 * identity plan is written by one launch over all events, and the launches of the general
 * plan that follow return at once unless some 256-event range was not sorted or held an
 * index out of range. */
int64_t cortex_pack_workspace_bytes(int64_t E, int64_t B);
int cortex_pack_plan(const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B, int64_t* offsets,
                     int64_t* order, int64_t* dst_rows, int64_t* rank, void* workspace, int64_t workspace_bytes,
                     int32_t* err_flag, int32_t* identity, int flags, hipStream_t stream);
#define CORTEX_PACK_CLEAR_ERR 1
/* cortex_pack_plan with a widening rider (see cortex_widen_int8): up to 8 int8 arrays widened
 * to bf16 by extra workgroups of the plan's first launch, on the CUs that the plan (a few
 * workgroups) leaves idle.  The plan itself is exactly cortex_pack_plan's. */
int cortex_pack_plan_widen(const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B, int64_t* offsets,
                           int64_t* order, int64_t* dst_rows, int64_t* rank, void* workspace,
                           int64_t workspace_bytes, int32_t* err_flag, int32_t* identity, int flags, int n_widen,
                           const void* const* widen_src, void* const* widen_dst, const int64_t* widen_count,
                           const int64_t* widen_frag_k, hipStream_t stream);

/* cortex_pack_plan without a workspace argument and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is a static device array of cortex_pack_noalloc_max_workspace_bytes()
 * (4 MiB) per GPU, held until the process ends; sizes with
 * cortex_pack_workspace_bytes(E, B) above it return -4 before any launch.  Every call on
 * one GPU uses that GPU's one array: calls that overlap on a GPU (concurrent streams)
 * race.  Outputs and semantics equal cortex_pack_plan's with identity == NULL. */
int64_t cortex_pack_noalloc_max_workspace_bytes(void);
int cortex_pack_plan_noalloc(const int64_t* batch_indices, int64_t s_bidx, int64_t E, int64_t B, int64_t* offsets,
                             int64_t* order, int64_t* dst_rows, int64_t* rank, int32_t* err_flag,
                             hipStream_t stream);

/* ---- a1 (+a2): fused spike tokenizer --------------------------------------
 * Replaces fused_tokenizer (cortex/kernels/tokenizer.py:177-249) and the eager
 * embedding sum of SpikeTokenizer.forward (cortex/models/tokenizer.py:90-93):
 *   out[r, :] = (neuron_emb[nid[e]] + time_emb[tb[e]]) + value_emb[val[e]]
 * evaluated left to right in the table dtype (f32 / bf16 / f16), where e is
 *   - r                        (order == NULL, offsets == NULL),
 *   - order[r]                 (CSR pack: order from cortex_pack_plan; rows
 *                              r >= *csr_end, if csr_end != NULL, are zero -- pass
 *                              &offsets[B] so that events dropped for an invalid
 *                              batch index never leave an unwritten order entry), or
 *   - order[offsets[b] + j]    for padded row r = b*E_max + j when offsets != NULL;
 *     rows j >= count_b are zero and mask[r] = (j < count_b), as the padded
 *     output of _pack_events (cortex/models/cortex.py:146-147,163-164).
 * identity (nullable): the plan's flag; when *identity != 0, order is not read and
 * order[x] is taken as x. */
int cortex_tokenize(int dtype, int64_t D, const void* neuron_emb, int64_t n_neuron, int64_t ld_neuron,
                    const void* time_emb, int64_t n_time, int64_t ld_time, const void* value_emb, int64_t n_value,
                    int64_t ld_value, const int64_t* neuron_ids, int64_t s_nid, const int64_t* time_bins,
                    int64_t s_tb, const int64_t* values, int64_t s_val, int64_t E, const int64_t* order,
                    const int64_t* csr_end, const int64_t* offsets, int64_t B, int64_t E_max, void* out,
                    int64_t ld_out, uint8_t* mask, const int32_t* identity, int32_t* err_flag,
                    hipStream_t stream);

/* ---- a1 + a3: tokens straight to the kv-projection operand -------------------
 * Replaces SpikeTokenizer.forward (cortex/models/tokenizer.py:90-93) followed by
 * CrossAttentionBlock.norm_kv (cortex/models/perceiver.py:67) in the model forward,
 * without storing the fp32 tokens:
 *   row r = LN((neuron_emb[nid[e]] + time_emb[tb[e]]) + value_emb[val[e]]) in bf16,
 *   e = order[r] (order NULL or *identity != 0: e = r), the sum in fp32 left to right, LN with
 *   gamma/beta/eps.  Rows r >= *csr_end (when csr_end is given) and rows with an index
 *   outside its table take x = 0 (LN gives beta); the latter OR 1 into err_flag.
 * fp32 tables, gamma, beta with 16-byte aligned rows; D in {256, 512, 768, 1024}. */
int cortex_tokenize_ln(int64_t D, const float* neuron_emb, int64_t n_neuron, int64_t ld_neuron, const float* time_emb,
                       int64_t n_time, int64_t ld_time, const float* value_emb, int64_t n_value, int64_t ld_value,
                       const int64_t* neuron_ids, int64_t s_nid, const int64_t* time_bins, int64_t s_tb,
                       const int64_t* values, int64_t s_val, int64_t E, const int64_t* order, const int32_t* identity,
                       const int64_t* csr_end, const float* gamma, const float* beta, float eps, void* out_bf16,
                       int64_t ld_out, int32_t* err_flag, hipStream_t stream);

/* ---- a2: pack existing token rows ------------------------------------------
 * Replaces the gather/scatter of _pack_events (cortex/models/cortex.py:150-164)
 * for already-tokenized (E, D) rows; same row mapping as cortex_tokenize. */
int cortex_pack_rows(int dtype, int64_t D, const void* src, int64_t ld_src, int64_t E, const int64_t* order,
                     const int64_t* csr_end, const int64_t* offsets, int64_t B, int64_t E_max, void* out,
                     int64_t ld_out, uint8_t* mask, hipStream_t stream);

/* ---- a7: INT8 per-channel weight quantisation ------------------------------
 * Replaces the weight scale of derive_scales (cortex/quantization/calibrate.py:154)
 * and the quantise step of QuantizedLinear.from_linear (calibrate.py:216-220):
 *   scale[n] = max(max_k |w[n,k]|, 1e-8) / 127   (written to scale_out)
 *   q[n,k]   = clamp(rint(w[n,k] / scale[n]), -127, 127)
 * When scale_in is not NULL it is used instead of the computed scale; when q is
 * NULL only the scales are computed (derive_scales). */
int cortex_quantize_int8(const float* w, int64_t N, int64_t K, int64_t ld_w, const float* scale_in,
                         float* scale_out, int8_t* q, int64_t ld_q, hipStream_t stream);

/* ---- a5/a6: per-row norm statistics ----------------------------------------
 * norm 1 (LayerNorm, cortex/models/perceiver.py:51-52): stats[2m] = mean,
 * stats[2m+1] = 1/sqrt(var + eps); norm 2 (RMSNorm,
 * cortex/kernels/fused_rmsnorm.py:102): stats[2m] = 0, stats[2m+1] = sqrt(mean(x^2) + eps). */
int cortex_row_stats(int64_t M, int64_t K, int x_dtype, const void* x, int64_t ld_x, int norm, float eps,
                     float* stats, hipStream_t stream);

/* ---- a8: LayerNorm written out ---------------------------------------------
 * Replaces nn.LayerNorm where its output is consumed by something other than a
 * linear, e.g. the encoder's final_norm feeding the behaviour head's own norm
 * (cortex/models/perceiver.py:158, cortex/models/cortex.py:37):
 *   out[m,k] = (x[m,k] - mean_m) * rstd_m * gamma[k] + beta[k]  (gamma/beta nullable). */
int cortex_layer_norm(int64_t M, int64_t K, int x_dtype, const void* x, int64_t ld_x, const void* gamma,
                      const void* beta, int gamma_dtype, float eps, int out_dtype, void* out, int64_t ld_out,
                      hipStream_t stream);

/* ---- a6: the norm half of a fused norm + linear, as bf16 rows --------------
 * The RMSNorm of rms_norm_linear (cortex/kernels/fused_rmsnorm.py:100-106:
 * ((x_f32 / sqrt(mean(x^2) + eps)) * gamma).to(bf16)) or a LayerNorm (norm = 1), for
 * the bf16 operand of the linear that follows; x fp32 or bf16, gamma/beta fp32 or bf16
 * (gamma_dtype), K in {256, 512, 768, 1024}.  The linear then runs on the bf16 GEMM. */
int cortex_norm_rows(int64_t M, int64_t K, int x_dtype, const void* x, int64_t ld_x, int norm, const void* gamma,
                     const void* beta, int gamma_dtype, float eps, void* out, int64_t ld_out, hipStream_t stream);
/* out[c, r] = in[r, c] for bf16 (R, C): rms_norm_linear's (K, N) weight
 * (fused_rmsnorm.py:239-245) as the (N, K) rows the GEMM streams.  Exact copies. */
int cortex_transpose_bf16(int64_t R, int64_t C, const void* in, int64_t ld_in, void* out, int64_t ld_out,
                          hipStream_t stream);
/* The RMSNorm gain of rms_norm_linear (fused_rmsnorm.py:223: (x / rms) * gamma) folded into
 * the weight's input columns, once per (weight, gamma) pair, as bf16 (N, K) rows:
 *   out[n, k] = bf16( float(w[n, k]) * gamma[k] )   (kn = 0, (N, K) rows: QuantizedLinear's
 *                                                    int8 weight or an nn.Linear weight)
 *   out[n, k] = bf16( float(w[k, n]) * gamma[k] )   (kn = 1, rms_norm_linear's (K, N) weight)
 * w int8, bf16 or fp32 (w_dtype); gamma fp32 or bf16.  cortex_norm_linear_fused with
 * norm 2 and gamma = NULL then applies the per-row 1 / rms to the fp32 accumulator. */
int cortex_fold_gain(int64_t N, int64_t K, const void* w, int w_dtype, int kn, int64_t ld_w, const void* gamma,
                     int gamma_dtype, void* out, int64_t ld_out, hipStream_t stream);
/* An (N, K) weight (int8, bf16 or fp32 rows: w_dtype 3 / 1 / 0) as bf16 in MFMA fragment
 * order, the layout of weight code 7: 1 KiB block (n16, k32) = n16 * (K / 32) + k32 holds rows
 * 16 n16 .. +15 and K 32 k32 .. +31 as 64 lanes x 8 values, lane l = row 16 n16 + l % 16,
 * K 32 k32 + 8 (l / 16) .. +7.  Values as cortex_convert writes them (int8 exact).  Built once
 * per weight, like the bf16 image of QuantizedLinear's dequantised weight (calibrate.py:
 * 225-228), for cortex_linear_residual_ln.  N % 16 == 0, K % 32 == 0, out (N * K bf16)
 * 16-byte aligned. */
int cortex_frag_weight(int64_t N, int64_t K, const void* w, int w_dtype, int64_t ld_w, void* out,
                       hipStream_t stream);

/* ---- a5/a8: LayerNorm rows to bf16 ----------------------------------------
 * Replaces nn.LayerNorm feeding a bf16 linear (cortex/models/perceiver.py:67-68,
 * 113,125,158; cortex/models/cortex.py:37), K in {256, 512, 768, 1024}:
 *   y = LN1(x) (gamma1/beta1/eps1), then y = LN2(y) when gamma2 or beta2 is given;
 *   written to out_bf16 (bf16) and/or out_f32.  fp32 x, gamma, beta (16-byte aligned). */
int cortex_ln_rows(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma1, const float* beta1,
                   float eps1, const float* gamma2, const float* beta2, float eps2, void* out_bf16, int64_t ld_bf16,
                   float* out_f32, int64_t ld_f32, hipStream_t stream);

/* ---- a7: INT8 weights widened to bf16 on the way ----------------------------
 * dst[i][e] = (bf16) src[i][e] for n <= 8 int8 arrays of count[i] elements (count[i] a
 * multiple of 16, both arrays 16-byte aligned): the dequantise step of
 * QuantizedLinear.forward (cortex/quantization/calibrate.py:227-228, q.float() before the
 * per-channel scale, which stays on the GEMM's accumulator), exact since every int8 value is a
 * bf16 value.  cortex_widen_int8 launches it on its own; the _widen forms of the LayerNorm row
 * kernels and of the tokenizer + LayerNorm run it in extra workgroups of their own launch (the
 * next block's weights ride along with the rows that feed it), otherwise exactly as
 * cortex_ln_rows / cortex_tokenize_ln.  The widened arrays must not overlap the kernel's
 * inputs or outputs.  frag_k (nullable): per array 0, or the row length K (a power of two from
 * 64) of an (N, K) weight to write in MFMA fragment order, the layout of weight code 7
 * (cortex_frag_weight), count a multiple of 16 K. */
int cortex_widen_int8(int n, const void* const* src, void* const* dst, const int64_t* count, const int64_t* frag_k,
                      hipStream_t stream);
int cortex_ln_rows_widen(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma1, const float* beta1,
                         float eps1, const float* gamma2, const float* beta2, float eps2, void* out_bf16,
                         int64_t ld_bf16, float* out_f32, int64_t ld_f32, int n_widen, const void* const* widen_src,
                         void* const* widen_dst, const int64_t* widen_count, const int64_t* widen_frag_k,
                         hipStream_t stream);
int cortex_tokenize_ln_widen(int64_t D, const float* neuron_emb, int64_t n_neuron, int64_t ld_neuron,
                             const float* time_emb, int64_t n_time, int64_t ld_time, const float* value_emb,
                             int64_t n_value, int64_t ld_value, const int64_t* neuron_ids, int64_t s_nid,
                             const int64_t* time_bins, int64_t s_tb, const int64_t* values, int64_t s_val, int64_t E,
                             const int64_t* order, const int32_t* identity, const int64_t* csr_end, const float* gamma,
                             const float* beta, float eps, void* out_bf16, int64_t ld_out, int32_t* err_flag,
                             int n_widen, const void* const* widen_src, void* const* widen_dst,
                             const int64_t* widen_count, const int64_t* widen_frag_k,
                             hipStream_t stream);

/* ---- a7: dtype conversion ---------------------------------------------------
 * out[i] = (out dtype) in[i]; int8 / f32 / bf16 / f16 in, f32 / bf16 out (bf16 by
 * round-to-nearest-even).  Builds the bf16 execution image of INT8 weights, which is
 * exact: every int8 value is a bf16 value (no reference counterpart; used by the
 * linear layers of cortex/quantization/calibrate.py:170-235). */
int cortex_convert(int in_dtype, const void* in, int out_dtype, void* out, int64_t n, hipStream_t stream);

/* ---- a5/a6/a7: fused norm + linear -----------------------------------------
 * Replaces rms_norm_linear (cortex/kernels/fused_rmsnorm.py:239-301),
 * QuantizedLinear.forward (cortex/quantization/calibrate.py:225-228) and the
 * LayerNorm -> Linear (-> GELU) (+ residual) chains of SelfAttentionBlock /
 * CrossAttentionBlock / BehaviorDecoder (cortex/models/perceiver.py:67-68,113-125;
 * cortex/models/cortex.py:37-53):
 *   a[m,k]   = x[m,k]                                  (norm 0)
 *            = (x[m,k]-mean_m)*rstd_m*gamma[k]+beta[k]   (norm 1, stats from cortex_row_stats)
 *            = (x[m,k]/rms_m)*gamma[k]                    (norm 2)
 *   a is rounded to the compute dtype (1 bf16 / 0 f32);
 *   acc[m,n] = sum_k a[m,k] * W[n,k]   (fp32 accumulation on MFMA)
 *   y[m,n]   = act(acc*w_scale[n] + bias[n]) + residual[(m % res_rows), n]
 * W: int8 (N,K) (w_layout 0) with w_scale, or bf16/f32 in (N,K) (layout 0) or
 * (K,N) (layout 1, the rms_norm_linear weight); a bf16 W may carry w_scale too
 * (the exact bf16 image of an int8 weight).  act: 0 none, 1 erf-GELU.
 * res_rows 0 means M (ordinary residual); a smaller value broadcasts a
 * batch-invariant residual such as the learned latents. */
int cortex_norm_linear(int64_t M, int64_t N, int64_t K, int x_dtype, const void* x, int64_t ld_x, int norm,
                       const float* stats, const void* gamma, const void* beta, int gamma_dtype, int compute,
                       int w_dtype, int w_layout, const void* w, int64_t ld_w, const float* w_scale,
                       int bias_dtype, const void* bias, int act, int res_dtype, const void* residual,
                       int64_t ld_res, int64_t res_rows, int out_dtype, void* out, int64_t ld_out,
                       hipStream_t stream);

/* Norm + linear in ONE launch (rms_norm_linear, cortex/kernels/fused_rmsnorm.py:130-233 and
 * :239-301, with QuantizedLinear's int8 weights, calibrate.py:170-235):
 *   y[m, :]  = bf16( x[m, :] / sqrt(mean_k x[m, k]^2 + eps) * gamma )             (norm 2, RMS)
 *            = bf16( (x[m, :] - mu) / sqrt(var + eps) * gamma + beta )             (norm 1, LayerNorm)
 *   out[m, n] = act( (sum_k y[m, k] w[n, k]) * w_scale[n] + bias[n] )
 * The row statistics are computed in the kernel's prologue from the x panel it stages in
 * LDS (no stats pass, no normalised rows in HBM).  x (M, K) bf16 with K a multiple of 64 up
 * to 512; w (N, K): w_dtype 1 bf16 or 3 int8 (widened exactly in the kernel); gamma/beta
 * fp32 or bf16 (gamma_dtype, beta ignored for RMS, optional for LayerNorm; gamma NULL with
 * RMS: no gain, the rows enter the MFMA as given and 1 / rms scales the fp32 accumulator,
 * for a weight that carries the gain, see cortex_fold_gain); w_scale, bias
 * optional fp32; act 0 or 1 (erf-GELU); out bf16 (1) or fp32 (0); N % 8 == 0; 16-byte
 * aligned rows (ld_w % 16 for int8); the weight (N x ld_w elements) under 2 GiB. */
int cortex_norm_linear_fused(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, int norm,
                             const void* gamma, const void* beta, int gamma_dtype, float eps, int w_dtype,
                             const void* w, int64_t ld_w, const float* w_scale, const float* bias, int act,
                             int out_dtype, void* out, int64_t ld_out, hipStream_t stream);

/* ---- a3/a4/a5/a8: attention ------------------------------------------------
 * Replaces sparse_cross_attention (cortex/kernels/sparse_xattn.py:340-434) and
 * the scaled_dot_product_attention calls of CrossAttentionBlock
 * (cortex/models/perceiver.py:75-80), SelfAttentionBlock (perceiver.py:121) and
 * BehaviorDecoder (cortex/models/cortex.py:49):
 *   out[b,h,i,:] = softmax_j(scale * q[b,h,i,:].k[b,h,j,:] | allowed) v[b,h,j,:]
 * Element (b,h,i,j) = base + b*s_b + h*s_h + i*s_l + d (q batch stride may be 0).
 * With kv_offsets (B+1), sample b's keys are CSR rows [kv_offsets[b], kv_offsets[b+1])
 * (row r at base + r*s_l + h*s_h), both ends clamped to [0, Lk] with Lk the number
 * of key rows of the view; otherwise Lk keys per sample.
 * Key j is allowed iff j < length (kv_lengths[b] when given), key_mask[b*km_sb + j]
 * != 0 (when given) and block_mask[b*bm_sb + (i/block_l)*n_kt + j/block_e] != 0
 * (when given; bm_sb 0 shares one tile mask across the batch).  Rows with no
 * allowed key are written as 0.  dtype: 1 bf16 or 0 f32; Dh <= 128. */
int cortex_attention(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dh, const void* q,
                     int64_t q_sb, int64_t q_sh, int64_t q_sl, const void* k, int64_t k_sb, int64_t k_sh,
                     int64_t k_sl, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sl,
                     const int64_t* kv_offsets, const int64_t* kv_lengths, const uint8_t* key_mask, int64_t km_sb,
                     const uint8_t* block_mask, int64_t bm_sb, int64_t n_qt, int64_t n_kt, int64_t block_l,
                     int64_t block_e, float scale, void* out, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                     hipStream_t stream);

/* build_temporal_block_mask (reference cortex/kernels/sparse_xattn.py:152-200) on the
 * device.  out[b * out_sb + qi * n_k + kj] = 1 iff query tile qi's window
 * [int(c(first)) - w, int(c(last)) + w], c(i) = float32(i) / n_latents * max_time_bins,
 * overlaps [min t, max t] of key tile kj's events (block_e events from the sample's
 * start).  offsets == NULL: one sample of E events (the reference's (n_q, n_k) mask);
 * otherwise (B+1) CSR offsets and a per-sample mask, key tiles past a sample's end 0.
 * Bit-exact with the reference's CPU loop. */
int cortex_temporal_block_mask(const int64_t* event_times, int64_t t_stride, int64_t E, const int64_t* offsets,
                               int64_t B, int64_t n_latents, int64_t max_time_bins, int64_t window_bins,
                               int64_t block_l, int64_t block_e, int64_t n_q, int64_t n_k, uint8_t* out,
                               int64_t out_sb, hipStream_t stream);

/* Self-attention with its QKV projection (SelfAttentionBlock, cortex/models/perceiver.py:
 * 113-121: qkv_proj on the norm_attn rows, split into heads, SDPA), one workgroup per
 * (head, sample), the projected q/k/v kept on chip:
 *   [q|k|v]_h[l] = xn[b*L + l] . W[{0,D,2D} + 64h + d]^T * w_scale (+ bias)
 *   out[b*L + l, 64h + d] = softmax_j(scale q_h[l] . k_h[j]) v_h[j]      (bf16)
 * xn (B*L, D) bf16 rows; w the (3D, D) weight with optional per-row scale and bias
 * (3D, fp32): w_dtype 1 the bf16 image, or 3 the int8 weight of the QuantizedLinear
 * (calibrate.py:170-235), widened exactly to bf16 inside the kernel (ld_w % 16 == 0).
 * Head dim 64 (D = 64 H), L <= 256, 16-byte aligned rows. */
int cortex_qkv_attention(int64_t B, int64_t L, int64_t D, int64_t H, const void* xn, int64_t ld_x, int w_dtype,
                         const void* w, int64_t ld_w, const float* w_scale, const float* bias, float scale, void* out,
                         int64_t ld_o, hipStream_t stream);

/* Residual linear followed by a LayerNorm (SelfAttentionBlock, cortex/models/perceiver.py:
 * 121-124: x = x + out_proj(attn); norm_mlp(x); and the cross-attention residual followed
 * by the first block's norm_attn):
 *   out[m, n] = res[(m % res_rows) * ld_res + n] + (sum_k x[m, k] w[n, k]) * w_scale[n] + bias[n]
 *   xn[m, :]  = LN(out[m, :]; gamma, beta, eps)   (bf16)
 * x (M, K) bf16; w (N, K): w_dtype 1 the weight's bf16 image, 3 the int8 weight of the
 * QuantizedLinear, widened exactly to bf16 inside the kernel (ld_w % 16 == 0), or 7 the
 * bf16 weight in fragment order (cortex_frag_weight; K 256 or 512, ld_w ignored), which
 * each wavefront streams straight into registers, bit-identical to w_dtype 1;
 * w_scale/bias optional, fp32; res/out fp32 (out may alias res: in-place residual
 * update); res_rows 0 means M.  N in {256, 512}, K % 64 == 0, 16-byte aligned rows. */
int cortex_linear_residual_ln(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, int w_dtype,
                              const void* w, int64_t ld_w, const float* w_scale, const float* bias, const float* res,
                              int64_t ld_res, int64_t res_rows, float* out, int64_t ld_out, const float* gamma,
                              const float* beta, float eps, void* xn, int64_t ld_xn, hipStream_t stream);

/* Opt-in W8A8 mode.  The reference derives a per-tensor activation scale per linear
 * (derive_scales, cortex/quantization/calibrate.py:145-150: 99th-percentile absmax / 127)
 * and never applies it (QuantizedLinear.forward dequantises the weight, :225-228); these
 * entry points apply it, for callers that accept int8 activations:
 *   q(y; s) = clamp(rint(y * (1 / s)), -127, 127)   (round half to even; 1/s in fp32)
 *
 * cortex_linear_residual_ln_i8: cortex_linear_residual_ln with the LayerNorm'd row
 * written as int8, xq[m, n] = q(LN(out[m, :])[n]; xq_scale); ld_xq a multiple of 16. */
int cortex_linear_residual_ln_i8(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, int w_dtype,
                                 const void* w, int64_t ld_w, const float* w_scale, const float* bias,
                                 const float* res, int64_t ld_res, int64_t res_rows, float* out, int64_t ld_out,
                                 const float* gamma, const float* beta, float eps, int8_t* xq, int64_t ld_xq,
                                 float xq_scale, hipStream_t stream);

/* cortex_linear_w8a8: y[m, n] = a_scale * w_scale[n] * sum_k x[m, k] w[n, k] + bias[n]
 * with x (M, K) int8 activations and w the (N, K) int8 weight of a QuantizedLinear, summed
 * exactly in int32 (v_mfma_i32_16x16x64_i8); act 1 applies the erf-GELU.  out_dtype 0:
 * fp32 out[m, n] = y (+ res[(m % res_rows), n], act 0 only; out may be res); out_dtype 3:
 * int8 out[m, n] = q(y; out_scale), the next linear's activation.  K % 128 == 0, N % 8 == 0;
 * 16-byte aligned rows (ld_x, ld_w multiples of 16, ld_out of 8). */
int cortex_linear_w8a8(int64_t M, int64_t N, int64_t K, const int8_t* x, int64_t ld_x, float a_scale, const int8_t* w,
                       int64_t ld_w, const float* w_scale, const float* bias, int act, const float* res,
                       int64_t ld_res, int64_t res_rows, void* out, int out_dtype, float out_scale, int64_t ld_out,
                       hipStream_t stream);

/* The rest of a self-attention block in the W8A8 mode (same q(.) as above):
 * cortex_qkv_attention_w8a8: cortex_qkv_attention with int8 xn rows at a_scale and the int8
 * qkv weight (exact int32 projection sums, a_scale * w_scale applied before the bf16
 * attention); out_dtype 1: bf16 o, 3: int8 o = q(o; out_scale) (out_proj's activation).
 * D a multiple of 128; ld_x, ld_w multiples of 16.
 * cortex_linear_residual_ln_w8a8: cortex_linear_residual_ln with int8 x rows at a_scale and
 * the int8 weight (N = 512, K % 128 == 0); xn bf16 (xn_dtype 1) or int8 = q(LN(out); xn_scale)
 * (xn_dtype 3).
 * cortex_ln_rows_i8: out = q(LN(x) * gamma + beta; out_scale) as int8 rows (K in {256, 512,
 * 768, 1024}; out 4-byte aligned, ld_out % 4 == 0). */
int cortex_qkv_attention_w8a8(int64_t B, int64_t L, int64_t D, int64_t H, const int8_t* xq, int64_t ld_x,
                              float a_scale, const int8_t* w, int64_t ld_w, const float* w_scale, const float* bias,
                              float scale, void* out, int out_dtype, float out_scale, int64_t ld_o,
                              hipStream_t stream);
int cortex_linear_residual_ln_w8a8(int64_t M, int64_t N, int64_t K, const int8_t* xq, int64_t ld_x, float a_scale,
                                   const int8_t* w, int64_t ld_w, const float* w_scale, const float* bias,
                                   const float* res, int64_t ld_res, int64_t res_rows, float* out, int64_t ld_out,
                                   const float* gamma, const float* beta, float eps, void* xn, int xn_dtype,
                                   float xn_scale, int64_t ld_xn, hipStream_t stream);
int cortex_ln_rows_i8(int64_t M, int64_t K, const float* x, int64_t ld_x, const float* gamma, const float* beta,
                      float eps, int8_t* out, int64_t ld_out, float out_scale, hipStream_t stream);

/* Behaviour head (BehaviorDecoder.forward, cortex/models/cortex.py:29-53) with its
 * batch-invariant factors folded: cortex_head_prep builds, once per parameter state,
 * the (32, D) bf16 matrix ac of rows a_{q,h} = W_k[h]^T q_h * log2(e)/sqrt(Dh) (rows
 * r = q*H + h < Q*H) and c_{h} = W_v[h]^T w_out[h] (rows 16 + r, h = r % H), from the
 * projected queries qv (Q, D) bf16, the kv weight image (2D, D) bf16 with optional
 * per-row scale s_kv (2D), and the output weight image (1, D) with optional scale.
 * Requires Q*H <= 16, Dh = D / H. */
int cortex_head_prep(const void* qv, int64_t ld_q, int64_t Q, int64_t H, int64_t D, const void* wkv,
                     const float* s_kv, int64_t ld_w, const void* wout, const float* s_out, void* ac,
                     hipStream_t stream);

/* cortex_behavior_head: out[b, q] (B, Q) fp32 from the fp32 latents x (B*L rows of D,
 * row b*L + l at x + (b*L + l) * ld_x): n_l = LN2(LN1(x_l)) (gamma/beta/eps each, rounded
 * to bf16), s = ac[r] . n_l, t = ac[16 + r] . n_l, out[b,q] = sum_h sum_l 2^s t / sum_l 2^s
 * over rows r = q*H + h -- the reference head's value up to rounding (softmax weights
 * sum to one, so V and out_proj commute with the sum over latents).  D in {256, 512,
 * 768}; rows and parameters 16-byte aligned; workspace of
 * cortex_behavior_head_workspace_bytes(B, L) bytes for the per-split partials. */
int cortex_behavior_head(const float* x, int64_t ld_x, int64_t B, int64_t L, int64_t D, int64_t Q, int64_t H,
                         const float* gamma1, const float* beta1, float eps1, const float* gamma2,
                         const float* beta2, float eps2, const void* ac, float* out, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream);

/* Bytes of the partials workspace cortex_behavior_head needs for B samples of L latents. */
int64_t cortex_behavior_head_workspace_bytes(int64_t B, int64_t L);

/* Masked-spike head (MaskedSpikeHead.forward, cortex/models/cortex.py:56-69, returned as
 * masked_spike_logits by CortexModel.forward(return_aux=True), :119-120):
 *   m_b = mean_l LN(x[b*L + l])          (LN skipped when gamma is null)
 *   out[b, n] = m_b . w[n] (* w_scale[n] for int8) + bias[n]
 * x: B*L fp32 rows of D (16-byte aligned, ld_x apart); w: (N, D) fp32, or int8 with its
 * per-row scale (QuantizedLinear, calibrate.py:225-228); bias optional.  pooled (B, D)
 * receives the mean rows when non-null (w may then be null: the mean alone).
 * D in {256, 512, 768, 1024}. */
int cortex_pooled_linear(const float* x, int64_t ld_x, int64_t B, int64_t L, int64_t D, const float* gamma,
                         const float* beta, float eps, int64_t N, int w_dtype, const void* w, int64_t ld_w,
                         const float* w_scale, const float* bias, float* pooled, float* out,
                         hipStream_t stream);

/* Streaming window assembly from device event pages.  No single reference
 * counterpart: it serves StreamingKVCache's role (cortex/cache/streaming.py:79-236)
 * with pages of raw events keyed by ABSOLUTE time bin, since the reference's window
 * time bins are relative to the window start (cortex/data/nlb.py:253-256), so cached
 * tokens would not be reusable.  pool: (num_pages, 3, page_events) int64 rows of
 * neuron id, absolute bin, value.  plan: (n_items, 4) int64 of (page, count,
 * first output row, bin shift); item i writes rows [dst, dst+count) of
 * out[f * field_stride + row] with the bin rewritten as bin - shift.  A malformed
 * item (page or rows out of range) writes nothing and sets bit 2 of *err (when
 * given).  Bit-exact copies. */
int cortex_gather_event_pages(const int64_t* pool, int64_t num_pages, int64_t page_events, const int64_t* plan,
                              int64_t n_items, int64_t* out, int64_t field_stride, int64_t out_rows, int32_t* err,
                              hipStream_t stream);

/* The page write of the same cache (reference StreamingKVCache.write,
 * cortex/cache/streaming.py:155-190, batched): plan (n_items, 3) int64 of (page,
 * count, first staged row); item i copies staged rows [s0, s0+count) of
 * src[f * field_stride + row] into page `page` of the pool.  A malformed item writes
 * nothing and sets bit 2 of *err (when given).  Bit-exact copies. */
int cortex_scatter_event_pages(const int64_t* src, int64_t field_stride, int64_t src_rows, const int64_t* plan,
                               int64_t n_items, int64_t* pool, int64_t num_pages, int64_t page_events, int32_t* err,
                               hipStream_t stream);

/* Residual linears for small row counts, K split across workgroups: the same results
 * as cortex_norm_linear with a residual (QuantizedLinear.forward plus the residual
 * add, cortex/quantization/calibrate.py:225-228, cortex/models/perceiver.py:121-125)
 * and as cortex_linear_residual_ln, up to the order of the fp32 sums.  K is cut into
 * `splits` slabs (K a multiple of 64 * splits); each slab's scaled partial product
 * goes to its fp32 (M, N) slab of the workspace, and the slabs are then summed in slab
 * order with bias and residual (row m % res_rows; out may be res).  The LayerNorm
 * variant also writes LN(out) * gamma + beta as bf16 rows (N in {256, 512, 768, 1024}).
 * x (M, K) and w (N, K) are bf16 rows; the workspace holds
 * cortex_splitk_workspace_bytes(M, N, splits) bytes, 16-byte aligned. */
int64_t cortex_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits);
int cortex_linear_residual_splitk(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, const void* w,
                                  int64_t ld_w, const float* w_scale, const float* bias, const float* res,
                                  int64_t ld_res, int64_t res_rows, float* out, int64_t ld_out, int64_t splits,
                                  void* workspace, int64_t workspace_bytes, hipStream_t stream);
int cortex_linear_residual_ln_splitk(int64_t M, int64_t N, int64_t K, const void* x, int64_t ld_x, const void* w,
                                     int64_t ld_w, const float* w_scale, const float* bias, const float* res,
                                     int64_t ld_res, int64_t res_rows, float* out, int64_t ld_out,
                                     const float* gamma, const float* beta, float eps, void* xn, int64_t ld_xn,
                                     int64_t splits, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* Host page table of that cache (no device work; not thread-safe, one caller per
 * table).  Replaces the Python bookkeeping of StreamingKVCache with the same policy
 * (cortex/cache/streaming.py:133-233): a lookup of a present key touches its page
 * (most recently used) and counts a hit, an absent key counts a miss; a write reuses
 * the key's page or allocates one, from the free list (last freed first) or by
 * evicting the least recently used page, records its event count and touches it;
 * evicting a session frees its pages in first-write order.  Keys are
 * (session id, first bin) with session ids chosen by the caller. */
int cortex_page_table_create(int64_t num_pages, void** table);
int cortex_page_table_destroy(void* table);
/* n page writes in order; page_ids[i] receives the page of entry i. */
int cortex_page_table_write(void* table, int64_t n, const int64_t* sessions, const int64_t* bin_starts,
                            const int64_t* n_events, int64_t* page_ids);
/* *page_id = the key's page (touched) or -1; *n_events its event count (0 if absent). */
int cortex_page_table_lookup(void* table, int64_t session, int64_t bin_start, int64_t* page_id, int64_t* n_events);
/* Gather plan of n_windows windows [window_starts[w], + window_bins): every page of
 * each window, in order, is looked up; items (capacity items_cap >= n_windows *
 * window_bins / bins_per_page rows of 4) receive (page, count, first output row,
 * window start) for the non-empty pages, offsets (n_windows + 1) the first output
 * row of each window.  If window w lacks pages, *missing_window = w, missing[0 ..
 * *n_missing) hold the first bins of its absent pages, and no window after w is
 * looked up; otherwise *missing_window = -1.  Replaces the per-page lookups of
 * StreamingKVCache.read (cortex/cache/streaming.py:133-153) for a batch of windows. */
int cortex_page_table_plan(void* table, int64_t n_windows, const int64_t* sessions, const int64_t* window_starts,
                           int64_t window_bins, int64_t bins_per_page, int64_t* items, int64_t items_cap,
                           int64_t* n_items, int64_t* offsets, int64_t* missing_window, int64_t* missing,
                           int64_t* n_missing);
/* StreamingKVCache.evict_session (cortex/cache/streaming.py:192-201): *freed = pages freed. */
int cortex_page_table_evict_session(void* table, int64_t session, int64_t* freed);
int cortex_page_table_stats(void* table, int64_t* hits, int64_t* misses, int64_t* pages_used);

#ifdef __cplusplus
}
#endif

#endif /* CORTEX_HIP_H_ */
