/*
 * shadowinfer_hip.h — C ABI of the MI355X (gfx950) quantized data plane.
 *
 * One shared library, libshadowinfer_hip.so, exports these entry points. They
 * replace the torch op chains of the reference's hot path (cited per entry as
 * file:line in ShadowInfer). Conventions:
 *
 *  - Every pointer argument named for data is a DEVICE pointer unless the
 *    comment says "host". Tables of bucket pointers (`buckets`) are HOST
 *    arrays of 16 device pointers: buckets[4*p + j], p = precision code
 *    (0 fp32, 1 fp16, 2 int8, 3 int4), j = 0 k, 1 v, 2 scale_k, 3 scale_v.
 *    Entries for absent buckets may be NULL.
 *  - Bucket memory uses the reference's tensor layouts exactly
 *    (shadowinfer/shadowkv/packed_kv_cache.py:137-218):
 *      fp32/fp16 : k,v [n, B, D]
 *      int8      : k,v [n, B, D] int8, scale [n, B, 1] in the input dtype
 *      int4      : k,v [n * ceil(B*D/2)] uint8 (offset-binary nibbles,
 *                  high nibble first), scale [n*B, D/g, 1] in the input dtype
 *    where n is the number of entries of that precision, ordered token-major.
 *  - Entries are token-heads; entry id e = t * H + h (token-major), which is
 *    the row-major flat index of the int8 [S, H] precision-code matrix.
 *  - The caller allocates every output and workspace. The library keeps no
 *    device allocations between calls and is reentrant; work is ordered on
 *    the given stream (a hipStream_t; NULL = the default stream).
 *  - Return value: 0 on success, non-zero on failure; si_last_error() then
 *    returns a thread-local message. Errors never fall back to other code.
 */
#ifndef SHADOWINFER_HIP_H
#define SHADOWINFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SI_ABI_VERSION 4

#define SI_OK 0
#define SI_ERR_INVALID 1
#define SI_ERR_HIP 2
#define SI_ERR_UNSUPPORTED 3

/* Element dtypes */
#define SI_DT_F32 0
#define SI_DT_F16 1
#define SI_DT_BF16 2

/* Precision codes: shadowinfer/shadowkv/precision_plan.py:20-26 */
#define SI_PREC_FP32 0
#define SI_PREC_FP16 1
#define SI_PREC_INT8 2
#define SI_PREC_INT4 3
#define SI_PREC_EVICTED 4

typedef void* si_stream_t;

/* Version of this ABI (SI_ABI_VERSION). No reference counterpart. */
int si_abi_version(void);

/* Self-check, no reference counterpart: converts every one of the 2^32 fp32
 * bit patterns to bf16 with the conversion the kernels use (gfx950's
 * v_cvt_pk_bf16_f32, NaN mapped to 0x7FC0) and compares with round-to-nearest-
 * even bit arithmetic. counts: device uint64[2], zeroed by the caller; adds
 * the mismatches of the two-value form to counts[0] and of the one-value form
 * to counts[1] (both stay 0 on a correct device). */
int si_check_bf16_convert(unsigned long long* counts, si_stream_t stream);

/* Test and tuning controls, no reference counterpart. Nothing in the library
 * reads the environment: these process-wide settings change a kernel choice
 * only when a caller sets them explicitly (tests that compare two code paths
 * of one operation, tile sweeps). Both start off.
 *
 * si_tune_gemm_plan: kind < 0 restores the automatic INT8 GEMM plan; kind >= 0
 * forces that internal tile kind (si_gemm.hip, enum Kind) and splits > 0 the
 * number of K splits of the tile kernels, for every later GEMM launch.
 * si_tune_attn_offset64: on != 0 makes the packed attention use its 64-bit
 * bucket addressing at every size (normally only caches of 2^31 bytes and
 * more do), so the two addressing paths can be compared on small caches. */
void si_tune_gemm_plan(int kind, int splits);
void si_tune_attn_offset64(int on);

/* Thread-local text of the last failure (empty string if none). Replaces the
 * TORCH_CHECK messages of shadowinfer/kernels/cpp/quantize_int4.cu:176-177. */
const char* si_last_error(void);

/* ---------------------------------------------------------------------- */
/* Precision plan                                                          */
/* ---------------------------------------------------------------------- */

/* Bytes of device workspace si_plan_scan needs for n_entries entries. */
size_t si_plan_workspace_bytes(int64_t n_entries);

/* Replaces the grouping of PrecisionPlan.from_codes
 * (shadowinfer/shadowkv/precision_plan.py:136-151) and of the evict
 * bookkeeping (shadowinfer/shadowkv/packed_kv_cache.py:679-737).
 * codes     : int8 [n_entries] (token-major); values outside 0..4 are absent
 * evict_mask: optional uint8 [n_entries]; non-zero forces a present entry absent
 * out_code  : int8 [n_entries], sanitized code (absent -> 4)
 * out_slot  : int32 [n_entries], position of the entry in its precision bucket
 *             (entries of one precision keep token-major order); -1 if absent
 * out_counts: int64 [5] device, entries per code 0..4 */
int si_plan_scan(const int8_t* codes, const uint8_t* evict_mask, int64_t n_entries,
                 int8_t* out_code, int32_t* out_slot, int64_t* out_counts,
                 void* workspace, size_t workspace_bytes, si_stream_t stream);

/* Replaces the flat-index build of PrecisionPlan.from_codes
 * (precision_plan.py:144-151): for each present entry e = t*H + h of code p,
 * flat_out[p][slot] = h*S + t (int64) and entry_out[p][slot] = e (int32).
 * flat_out / entry_out: HOST arrays of 4 device pointers (NULL to skip). */
int si_plan_scatter(const int8_t* code, const int32_t* slot, int64_t S, int64_t H,
                    int64_t* const* flat_out, int32_t* const* entry_out,
                    si_stream_t stream);

/* si_plan_scan and si_plan_scatter in one pass over S*H entries (one
 * counting launch and one launch that scans and fills the lists), for the
 * rescan of PackedKVCache.evict (shadowinfer/shadowkv/packed_kv_cache.py:
 * 679-737), whose new buckets are not known before the scan.
 * flat_out: HOST array of 4 device int64 lists; flat_capacity: HOST int64[4],
 * the rows each list holds (an evict passes the old bucket sizes, which bound
 * the new ones); slots at or past a list's capacity are not written.
 * Workspace: si_plan_workspace_bytes(S * H). */
int si_plan_scan_lists(const int8_t* codes, const uint8_t* evict_mask, int64_t S, int64_t H,
                       int8_t* out_code, int32_t* out_slot, int64_t* out_counts,
                       int64_t* const* flat_out, const int64_t* flat_capacity, void* workspace,
                       size_t workspace_bytes, si_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Packed KV cache                                                         */
/* ---------------------------------------------------------------------- */

/* Replaces PackedKVCache._do_pack_with_plan (packed_kv_cache.py:222-365),
 * including Quantizer.quantize_int8/int4 (utils/quantization.py:120-178) and
 * _pack_int4_rows (packed_kv_cache.py:367-388).
 * k, v: [B, H, S, D] contiguous, dtype SI_DT_*; group: effective int4 group
 * size (must divide D); code/slot: from si_plan_scan. Writes every bucket. */
int si_kv_pack(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t S,
               int64_t D, int64_t group, const int8_t* code, const int32_t* slot,
               void* const* buckets, si_stream_t stream);

/* si_kv_pack in bucket order: flat = HOST array of 4 device int64 lists
 * (flat[p][slot] = h*S + t, the plan's flat_indices), counts = HOST int64[5]
 * (entries per code 0..4, summing to S*H). Each block quantizes one
 * precision and writes its bucket rows contiguously. Same buckets as
 * si_kv_pack (which it uses for shapes the row kernels do not cover). */
int si_kv_pack_flat(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t S,
                    int64_t D, int64_t group, const int8_t* code, const int32_t* slot,
                    const int64_t* const* flat, const int64_t* counts, void* const* buckets,
                    si_stream_t stream);

/* Fused form of ShadowKVAgent._compress_kv_with_plan
 * (shadowinfer/shadowkv/shadowkv_agent.py:1698-1809) and si_kv_pack: one
 * pass over K/V writes the buckets (as si_kv_pack) and the dense working
 * copy out_k/out_v [B, H, S, D] in `dtype`: fp32 entries keep their values,
 * fp16 entries are rounded to fp16 and back, int8/int4 entries hold their
 * integer codes (not dequantized), other codes are 0. Entries e with
 * reuse_mask[e] != 0 (uint8 [S*H], may be NULL) take the rows of
 * k_prev/v_prev instead (both required when reuse_mask is given). */
int si_kv_pack_copy(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t S,
                    int64_t D, int64_t group, const int8_t* code, const int32_t* slot,
                    void* const* buckets, const void* k_prev, const void* v_prev,
                    const uint8_t* reuse_mask, void* out_k, void* out_v, si_stream_t stream);


/* Replaces PackedKVCache.unpack (packed_kv_cache.py:535-577) and
 * _dequantize_int4_bucket (636-656). Writes every element of out_k/out_v
 * ([B, H, S, D] fp32), absent entries as +0.0. scale_dtype: dtype of the
 * stored scales. */
int si_kv_unpack(const int8_t* code, const int32_t* slot, const void* const* buckets,
                 int scale_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                 int64_t group, float* out_k, float* out_v, si_stream_t stream);

/* si_kv_unpack in bucket order: flat = HOST array of 4 device int64 lists,
 * flat[p][slot] = h*S + t of the entries of precision p in slot order (the
 * plan's flat_indices, precision_plan.py:144-151, or si_plan_scatter);
 * counts = HOST int64[5], entries per code 0..4 (summing to S*H). Each
 * block decodes one precision and reads its bucket contiguously; entries of
 * code 4 are written as zeros. Same output as si_kv_unpack (which it uses
 * for shapes other than D in {64, 128} with 16-byte aligned outputs). */
int si_kv_unpack_flat(const int8_t* code, const int32_t* slot, const int64_t* const* flat,
                      const int64_t* counts, const void* const* buckets, int scale_dtype,
                      int64_t B, int64_t H, int64_t S, int64_t D, int64_t group, float* out_k,
                      float* out_v, si_stream_t stream);

/* Replaces the copy loop of PackedKVCache.apply_reuse_mask
 * (packed_kv_cache.py:791-852). For each present entry (t,h) of the current
 * cache with mask[t*H+h] != 0: if t < S_prev and the previous cache holds it
 * with the same precision, its data row and scale row(s) are copied from the
 * previous bucket; if the previous cache holds it with another precision,
 * stats[1] is incremented. stats (optional, int64 [2] device, zeroed by the
 * caller): applied, skipped_precision. */
int si_kv_reuse(const int8_t* cur_code, const int32_t* cur_slot, void* const* cur_buckets,
                int64_t S, const int8_t* prev_code, const int32_t* prev_slot,
                const void* const* prev_buckets, int64_t S_prev, const uint8_t* mask,
                int64_t H, int64_t B, int64_t D, int64_t group, int scale_dtype,
                int64_t* stats, si_stream_t stream);

/* Replaces the index_select compaction of PackedKVCache.evict
 * (packed_kv_cache.py:698-737): every entry present in new_code is copied from
 * old bucket row old_slot to new bucket row new_slot (same precision). */
int si_kv_compact(const int8_t* old_code, const int32_t* old_slot,
                  const void* const* old_buckets, const int8_t* new_code,
                  const int32_t* new_slot, void* const* new_buckets, int64_t n_entries,
                  int64_t B, int64_t D, int64_t group, int scale_dtype, si_stream_t stream);

/* si_kv_reuse in bucket order: walks the current cache's per-precision lists
 * cur_flat[p] (h*S + t in slot order, cur_counts HOST int64[5] entries each;
 * the plan's flat_indices, shadowinfer/shadowkv/precision_plan.py:144-151), one
 * precision per block, so destination rows are contiguous. Same copies and
 * stats as si_kv_reuse. */
int si_kv_reuse_flat(const int64_t* const* cur_flat, const int64_t* cur_counts,
                     void* const* cur_buckets, int64_t S, const int8_t* prev_code,
                     const int32_t* prev_slot, const void* const* prev_buckets, int64_t S_prev,
                     const uint8_t* mask, int64_t H, int64_t B, int64_t D, int64_t group,
                     int scale_dtype, int64_t* stats, si_stream_t stream);

/* si_kv_compact in bucket order: walks the new plan's per-precision lists
 * new_flat[p] (new_counts HOST int64[5]); each destination row is copied from
 * old bucket row old_slot[t*H + h]. Precisions whose new bucket pointer is NULL
 * are left alone (their bucket is kept as it is). */
int si_kv_compact_flat(const int32_t* old_slot, const void* const* old_buckets,
                       const int64_t* const* new_flat, const int64_t* new_counts,
                       void* const* new_buckets, int64_t S, int64_t H, int64_t B, int64_t D,
                       int64_t group, int scale_dtype, si_stream_t stream);

/* PackedKVCache.evict (packed_kv_cache.py:666-740) over the OLD grouping's
 * lists, in two passes and without a token-order rescan of the codes. The
 * old lists old_flat[p] (h*S + t per old slot, old_counts HOST int64[4]) are
 * cut into chunks of consecutive old slots of one precision;
 * si_kv_evict_chunks(old_counts) is the number of chunks (-1 on bad sizes)
 * and si_kv_evict_chunk_words() the uint64 words of survivor bits per chunk.
 *
 * si_kv_evict_count: chunk_counts[j] (int32) = survivors of chunk j, and
 * chunk_bits (chunks * words) their bit masks; new_code[e] = the old code, or
 * 4 where evict_mask[e] != 0 or the entry was absent (code outside 0..3);
 * new_slot[e] = -1 for every entry that is not kept. The caller reads
 * chunk_counts to size the new buckets: the new size of precision p is the
 * sum over its chunks.
 *
 * si_kv_evict_flat: every kept entry gets the new slot (survivors in the
 * earlier chunks of its precision) + (its rank in its chunk), i.e. the stable
 * in-bucket compaction; writes new_slot[e], new_flat[p][slot] (lists may be
 * NULL) and, for precisions whose new bucket pointer is set, the K/V rows
 * and scales. NULL new bucket pointers leave the precision's rows alone (the
 * caller keeps the bucket when nothing of it was evicted). new_counts (HOST
 * int64[4]) bound every slot written. */
int64_t si_kv_evict_chunks(const int64_t* old_counts);
int64_t si_kv_evict_chunk_words(void);
int si_kv_evict_count(const int8_t* old_code, const int64_t* const* old_flat,
                      const int64_t* old_counts, const uint8_t* evict_mask, int64_t S, int64_t H,
                      int8_t* new_code, int32_t* new_slot, int32_t* chunk_counts,
                      uint64_t* chunk_bits, si_stream_t stream);
int si_kv_evict_flat(const int64_t* const* old_flat, const int64_t* old_counts,
                     const int32_t* chunk_counts, const uint64_t* chunk_bits, int64_t S, int64_t H,
                     const void* const* old_buckets, int64_t* const* new_flat,
                     const int64_t* new_counts, void* const* new_buckets, int32_t* new_slot,
                     int64_t B, int64_t D, int64_t group, int scale_dtype, si_stream_t stream);

/* Bytes of device workspace si_attn_packed_fwd needs (per-head slot lists). */
size_t si_attn_workspace_bytes(int64_t H, int64_t S_kv);

/* Replaces unpack() -> softmax(q k^T * sm_scale) v with no mask
 * (shadowinfer/models/simple_diffusion_llm.py:165-169) as one fused kernel
 * that dequantizes packed K/V tiles into LDS; the dense K/V never exist.
 * Semantic neighbour of shadowinfer/kernels/__init__.py:473-537.
 * q: [B, H, S_q, D], q_dtype SI_DT_BF16 or SI_DT_F16, 16-byte aligned; D = 64
 * or 128; group: int4 group size (a multiple of D/16 dividing D).
 * out: [B, H, S_q, D] in out_dtype (SI_DT_F32 matches unpack()'s fp32 K/V),
 * 16-byte aligned.
 * workspace: si_attn_workspace_bytes(H, S_kv) bytes, 16-byte aligned. */
int si_attn_packed_fwd(const void* q, int q_dtype, int64_t B, int64_t H, int64_t S_q,
                       int64_t D, const int8_t* code, const int32_t* slot,
                       const void* const* buckets, int scale_dtype, int64_t S_kv,
                       int64_t group, float sm_scale, void* out, int out_dtype,
                       void* workspace, size_t workspace_bytes, si_stream_t stream);

/* si_attn_packed_fwd writing token-major out [B, S_q, H, D]: the
 * attn.transpose(1, 2).reshape(B, S, H * D) layout the output projection
 * reads (shadowinfer/models/diffusion_llama.py:390-391). */
int si_attn_packed_fwd_tokens(const void* q, int q_dtype, int64_t B, int64_t H, int64_t S_q,
                              int64_t D, const int8_t* code, const int32_t* slot,
                              const void* const* buckets, int scale_dtype, int64_t S_kv,
                              int64_t group, float sm_scale, void* out, int out_dtype,
                              void* workspace, size_t workspace_bytes, si_stream_t stream);

/* The per-head slot lists si_attn_packed_fwd builds on every call (tiles of
 * one precision per head) depend only on code and slot, i.e. on the plan:
 * build them once into lists (si_attn_workspace_bytes(H, S_kv) bytes,
 * 16-byte aligned) and reuse them for every cache packed with that plan. */
int si_attn_build_lists(const int8_t* code, const int32_t* slot, int64_t H, int64_t S_kv,
                        void* lists, size_t lists_bytes, si_stream_t stream);

/* si_attn_packed_fwd (token_major == 0: out [B, H, S_q, D]) or
 * si_attn_packed_fwd_tokens (token_major != 0: out [B, S_q, H, D]) over lists
 * built by si_attn_build_lists. */
int si_attn_packed_fwd_built(const void* q, int q_dtype, int64_t B, int64_t H, int64_t S_q,
                             int64_t D, const void* lists, size_t lists_bytes,
                             const void* const* buckets, int scale_dtype, int64_t S_kv,
                             int64_t group, float sm_scale, void* out, int out_dtype,
                             int token_major, si_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Quantizer                                                               */
/* ---------------------------------------------------------------------- */

/* Quantizer.quantize_int8 over rows of D (utils/quantization.py:120-142).
 * q: int8 [rows, D]; scale: [rows] in dtype. */
int si_quant_rows_i8(const void* x, int dtype, int64_t rows, int64_t D, int8_t* q,
                     void* scale, si_stream_t stream);

/* Quantizer.quantize_int4 (utils/quantization.py:144-178).
 * q: int8 [rows, D]; scale: [rows, D/group] in dtype. */
int si_quant_rows_i4(const void* x, int dtype, int64_t rows, int64_t D, int64_t group,
                     int8_t* q, void* scale, si_stream_t stream);

/* _pack_int4_rows (packed_kv_cache.py:367-388) / Quantizer.pack_int4
 * (utils/quantization.py:248-277) / kernels._pack_int4 (kernels/__init__.py:
 * 382-402): rows of L int8 codes -> rows of ceil(L/2) bytes. */
int si_int4_pack_rows(const int8_t* q, int64_t rows, int64_t L, uint8_t* out,
                      si_stream_t stream);

/* Quantizer.unpack_int4 (utils/quantization.py:279-318) / kernels._unpack_int4
 * (kernels/__init__.py:405-420): rows of row_bytes bytes -> rows of L codes. */
int si_int4_unpack_rows(const uint8_t* in, int64_t rows, int64_t row_bytes, int64_t L,
                        int8_t* out, si_stream_t stream);

/* Quantizer.dequantize_int8 / dequantize_int4 (utils/quantization.py:180-219):
 * out[r, d] = float(q[r, d]) * float(scale[r, d / group]). */
int si_dequant_rows(const int8_t* q, const void* scale, int scale_dtype, int64_t rows,
                    int64_t D, int64_t group, float* out, si_stream_t stream);

/* ---------------------------------------------------------------------- */
/* INT8 FFN linear                                                         */
/* ---------------------------------------------------------------------- */

/* INT8Linear.from_linear (ffn_optimizer/int8_linear.py:65-82):
 * w fp32 [N, K] -> qweight int8 [N, K], scale fp32 [N]. The quantized weight
 * keeps nn.Linear's [N, K] layout (K contiguous, the MFMA fragment layout);
 * the reference's stored [K, N] tensor is its transpose. */
int si_weight_quant_i8(const float* w, int64_t N, int64_t K, int8_t* qweight,
                       float* scale, si_stream_t stream);

/* INT8Linear.forward prologue (int8_linear.py:96-98): per-row dynamic
 * symmetric int8, clamp +-127, scale floor 1e-8. x [M, K] in dtype. */
int si_act_quant_i8(const void* x, int dtype, int64_t M, int64_t K, int8_t* q,
                    float* scale, si_stream_t stream);

/* Bytes of device workspace the GEMM entry points need for this shape (split-K
 * partial sums; 0 when the shape runs without splitting). */
size_t si_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* torch._int_mm (int8_linear.py:102): c[m, n] = sum_k a[m, k] * b[n, k],
 * a int8 [M, K], b int8 [N, K] (the weight in [N, K] layout), c int32 [M, N],
 * exact. */
int si_gemm_i8i8_i32(const int8_t* a, const int8_t* b, int64_t M, int64_t N, int64_t K,
                     int32_t* c, void* workspace, size_t workspace_bytes, si_stream_t stream);

/* _int_mm + epilogue (int8_linear.py:102-115): out[m, n] =
 * T(float(acc) * (sx[m] * sw[n]) [+ bias[n]]), T = out_dtype, b int8 [N, K].
 * bias optional. */
int si_gemm_i8_dequant(const int8_t* a, const float* sx, const int8_t* b, const float* sw,
                       const float* bias, int64_t M, int64_t N, int64_t K, void* out,
                       int out_dtype, void* workspace, size_t workspace_bytes,
                       si_stream_t stream);

/* si_gemm_i8_dequant followed by the decoder layer's residual add
 * (models/diffusion_llama.py:421-423, hidden = residual + mlp(...)):
 * out = T(residual + T(float(acc) * (sx * sw) [+ bias])), residual [M, N] in
 * out_dtype. out may be the residual buffer itself (an in-place add). */
int si_gemm_i8_dequant_add(const int8_t* a, const float* sx, const int8_t* b, const float* sw,
                           const float* bias, const void* residual, int64_t M, int64_t N,
                           int64_t K, void* out, int out_dtype, void* workspace,
                           size_t workspace_bytes, si_stream_t stream);

/* Workspace bytes of si_int8_linear_forward (quantized activations, their
 * scales and the GEMM workspace). */
size_t si_int8_linear_workspace_bytes(int64_t M, int64_t K, int64_t N);

/* Whole INT8Linear.forward on a 2-D input (int8_linear.py:88-115):
 * activation quantization, int8 GEMM, epilogue. qweight int8 [N, K];
 * out [M, N] in dtype. */
int si_int8_linear_forward(const void* x, int dtype, int64_t M, int64_t K, int64_t N,
                           const int8_t* qweight, const float* sw, const float* bias,
                           void* out, void* workspace, size_t workspace_bytes,
                           si_stream_t stream);

/* si_int8_linear_forward followed by the residual add of the decoder layer
 * (diffusion_llama.py:421-423): out = T(residual + T(INT8Linear(x))),
 * residual [M, N] in dtype; out may be the residual buffer itself. Same
 * workspace as si_int8_linear_forward. */
int si_int8_linear_forward_add(const void* x, int dtype, int64_t M, int64_t K, int64_t N,
                               const int8_t* qweight, const float* sw, const float* bias,
                               const void* residual, void* out, void* workspace,
                               size_t workspace_bytes, si_stream_t stream);

/* Size of the device scratch array of si_int8_linear_forward_noalloc (one
 * per device, held until the process ends). */
#define SI_INT8_LINEAR_SCRATCH_BYTES ((size_t)32 << 20)

/* No counterpart in the reference: si_int8_linear_forward for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results, no
 * workspace argument: the workspace is a library-owned device array of
 * SI_INT8_LINEAR_SCRATCH_BYTES per device, so shapes whose
 * si_int8_linear_workspace_bytes(M, K, N) exceeds it are rejected
 * (SI_ERR_INVALID). Allocates nothing. The first call on a device looks the
 * array up (call it once before capturing). Calls that overlap on one device
 * (other streams, other threads) share the array and race: order them. */
int si_int8_linear_forward_noalloc(const void* x, int dtype, int64_t M, int64_t K, int64_t N,
                                   const int8_t* qweight, const float* sw, const float* bias,
                                   void* out, si_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Paged KV store                                                          */
/* ---------------------------------------------------------------------- */

/* Replaces the row quantization and page write of PagedKVStore.append and
 * rewrite_tokens (shadowinfer/shadowkv/paged_kv_store.py:189-212, 248-307,
 * 407-447): tokens t0 .. t0+take-1 of k, v [B, H, T, D] (`dtype`) go to rows
 * offset .. offset+take-1 of a page of `capacity` rows per (b, h).
 * page: HOST array of 4 device pointers {k, v, scale_k, scale_v}:
 *   precision 0 ("fp32" page): k, v [B, H, capacity, D] in `dtype` (a copy)
 *   precision 1: k, v [B, H, capacity, D] fp16
 *   precision 2: k, v int8 [B, H, capacity, D]; scales [B, H, capacity, 1] in `dtype`
 *   precision 3: k, v uint8 [B, H, capacity, ceil(D/2)] (code + 8, high
 *                nibble first); scales [B, H, capacity, D/group, 1] in `dtype`
 * The row arithmetic is si_kv_pack's, so page rows equal packed-cache rows. */
int si_page_write(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t T,
                  int64_t D, int64_t t0, int64_t take, int precision, int64_t group,
                  void* const* page, int64_t capacity, int64_t offset, si_stream_t stream);

/* si_page_write for a run of n_pages fresh pages allocated page-major (page i
 * at pages[x] + i * its bytes per page, each page [B, H, capacity, ...]): tokens
 * t0 .. t0 + n_pages * capacity - 1 fill pages 0 .. n_pages - 1 in order, as
 * n_pages appends of whole pages would (paged_kv_store.py:248-307). */
int si_page_write_pages(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t T,
                        int64_t D, int64_t t0, int64_t n_pages, int precision, int64_t group,
                        void* const* pages, int64_t capacity, si_stream_t stream);

/* Replaces PagedKVStore.gather / _decode (paged_kv_store.py:326-405): every
 * page of the device table (int64 [n_pages, 9] rows {precision, dtype, k, v,
 * scale_k, scale_v, start token, tokens, capacity}; dtype = the page's input
 * dtype SI_DT_*, in which its scales and "fp32" payloads are stored, so pages
 * of one store may differ) decoded into fp32 out_k/out_v [B, H, S, D] at its
 * start token; rows no page covers are left as they are (the caller zeroes
 * them). */
int si_page_gather(const int64_t* table, int64_t n_pages, int64_t B, int64_t H, int64_t S,
                   int64_t D, int64_t group, float* out_k, float* out_v, si_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Rate-distortion admission                                               */
/* ---------------------------------------------------------------------- */

/* Replaces kv_sensitivity (shadowinfer/shadowkv/rd_allocator.py:47-61):
 * k, v [B, H, S, D] in `dtype`; out [S, H] in `dtype`,
 * out[t, h] = (amax_{b,d}|k|^2 + amax_{b,d}|v|^2) / 2 with every operation
 * rounded to `dtype` (NaN propagates). */
int si_kv_sensitivity(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t S,
                      int64_t D, void* out, si_stream_t stream);

/* Bytes of device workspace si_admit_codes needs for n_entries = S * H. */
size_t si_admit_workspace_bytes(int64_t n_entries);

/* Replaces admit_codes (shadowinfer/shadowkv/rd_allocator.py:190-318) and
 * predict_codes_bytes (:173-188).
 * codes, out_codes: int8 [S, H] (token-major; out_codes may not alias codes)
 * importance      : fp32 [S, H]
 * sensitivity     : fp32 [S, H], or NULL to rank by importance alone
 * protected_mask  : uint8 [S, H] (non-zero = never touched), or NULL
 * sink_tokens     : tokens t < sink_tokens are never touched
 * budget_bytes    : applied when use_budget != 0 (any value); otherwise the
 *                   codes are copied and only their bytes are summed
 * costs           : HOST int64 [5], bytes of one token-head per code
 *                   (int(entry_bytes(...)), rd_allocator.py:26-44)
 * result          : device int64 [3]: predicted bytes, newly evicted entries,
 *                   1 if a code outside 0..4 was seen (then nothing is admitted)
 * workspace       : 256-byte aligned, si_admit_workspace_bytes(S * H) bytes */
int si_admit_codes(const int8_t* codes, int8_t* out_codes, int64_t S, int64_t H,
                   const float* importance, const float* sensitivity,
                   const uint8_t* protected_mask, int64_t sink_tokens, int64_t budget_bytes,
                   int use_budget, int allow_eviction, const int64_t* costs, int64_t* result,
                   void* workspace, size_t workspace_bytes, si_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Denoising step of a Llama-shaped diffusion LM (row kernels)             */
/* ---------------------------------------------------------------------- */

/* DiffusionLlamaRMSNorm (shadowinfer/models/diffusion_llama.py:311-321) over
 * rows of K (K % 8 == 0, K <= 16384), following the reference's op chain
 * x / sqrt(mean(x^2) + eps) * w in T = dtype with every op rounded to T:
 * var = T(mean(T(x^2))) (fp32 sum), r = T(sqrt(T(var + eps))),
 * y = T(T(x / r) * w). x [M, K], weight [K] in dtype. Outputs (each optional,
 * at least one): y [M, K] in dtype; q int8 [M, K] + scale fp32 [M], the
 * INT8Linear activation quantization of y
 * (shadowinfer/ffn_optimizer/int8_linear.py:96-98), identical to
 * si_act_quant_i8 on y. */
int si_rmsnorm_rows(const void* x, int dtype, int64_t M, int64_t K, const void* weight,
                    float eps, void* y, int8_t* q, float* scale, si_stream_t stream);

/* The residual add of DiffusionLlamaDecoderLayer.forward
 * (shadowinfer/models/diffusion_llama.py:421-422) fused with the next
 * RMSNorm: x_out = T(x + residual) [M, K], then si_rmsnorm_rows on x_out
 * (same optional outputs y, q, scale). */
int si_add_rmsnorm_rows(const void* x, const void* residual, int dtype, int64_t M, int64_t K,
                        const void* weight, float eps, void* x_out, void* y, int8_t* q,
                        float* scale, si_stream_t stream);

/* RoPE and head split of DiffusionLlamaAttention.forward
 * (shadowinfer/models/diffusion_llama.py:362-373): qkv [B*S, 3*H*D] (q | k | v)
 * -> q, k, v [B, H, S, D]; q and k rotated as q * cos + rotate_half(q) * sin
 * in dtype (each product rounded, then the sum) with the rotate-half tables
 * cos_table, sin_table [S, D] (diffusion_llama.py:505-514). D = 64 or 128;
 * all pointers 16-byte aligned. k and v both NULL: only q is written (K and V
 * then go into the packed cache through si_kv_pack_rope_flat). */
int si_rope_split(const void* qkv, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
                  const void* cos_table, const void* sin_table, void* q, void* k, void* v,
                  si_stream_t stream);

/* si_rope_split's K and V rows packed straight into the buckets: the same
 * bytes as si_rope_split followed by si_kv_pack_flat on its k and v (the
 * attention layer's pack, pytorch_backend.py:521-548, on the post-RoPE K/V of
 * diffusion_llama.py:362-373), reading each K/V row from the projection
 * output qkv [B*S, 3*H*D] (q | k | v column blocks) and rotating K on the way.
 * dtype bf16 or fp16 (the buckets' scale dtype too); D = 64 or 128; group a
 * multiple of 8 dividing D with group/8 a power of two; qkv, cos_table and
 * sin_table 16-byte aligned. flat, counts and buckets as for si_kv_pack_flat. */
int si_kv_pack_rope_flat(const void* qkv, const void* cos_table, const void* sin_table,
                         int dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t group,
                         const int8_t* code, const int32_t* slot, const int64_t* const* flat,
                         const int64_t* counts, void* const* buckets, si_stream_t stream);

/* DiffusionLlamaMLP's silu(gate) * up (shadowinfer/models/diffusion_llama.py:332-333)
 * and the down INT8Linear's activation quantization (int8_linear.py:96-98):
 * gate_up [M, 2F] (gate | up) in dtype; h = T(T(silu(g)) * u) [M, F]
 * (optional) with silu(g) = g / (1 + expf(-g)) in fp32 as torch computes it,
 * q int8 [M, F], scale fp32 [M]. F % 8 == 0, F <= 16384. For bf16 and fp16 the
 * first call on a device also fills a 256 KB silu table in module memory. */
int si_swiglu_quant(const void* gate_up, int dtype, int64_t M, int64_t F, void* h, int8_t* q,
                    float* scale, si_stream_t stream);

/* Per-position token and confidence of schedule_round
 * (shadowinfer/execution/block_decoding.py:146-147): probs = softmax(logits)
 * in the logits' dtype T, (confidence, tokens) = probs.max(-1).
 * confidence[m] = T(1 / s), s = sum_v expf(l_v - l_max) in fp32, written in T
 * (the logits' dtype); tokens[m] = the first v whose rounded probability
 * T(expf(l_v - l_max) / s) equals it. A row with a NaN or +inf logit, or only
 * -inf logits, gives confidence NaN and token 0. logits [M, V]. */
int si_row_argmax_conf(const void* logits, int dtype, int64_t M, int64_t V, int64_t* tokens,
                       void* confidence, si_stream_t stream);

/* Bytes of device workspace si_reuse_drift needs (independent of n). */
size_t si_reuse_drift_workspace_bytes(int64_t n);

/* The two reductions of the step-reuse drift gate
 * (shadowinfer/execution/step_reuse.py:71-80), ||hidden - hidden_in|| and
 * ||hidden_in|| before their square roots: out[0] = sum T(h - h_in)^2,
 * out[1] = sum h_in^2, fp32 accumulation (device float[2]); h, h_in: n
 * elements in dtype T, 16-byte aligned. Deterministic for a given n. */
int si_reuse_drift(const void* hidden, const void* hidden_in, int dtype, int64_t n, float* out,
                   void* workspace, size_t workspace_bytes, si_stream_t stream);

/* The reused block output of DiffusionTransformerBlock.forward
 * (shadowinfer/models/simple_diffusion_llm.py:104):
 * out = T(hidden_out + T(hidden - hidden_in)), n elements in dtype T. */
int si_reuse_apply(const void* hidden, const void* hidden_in, const void* hidden_out, int dtype,
                   int64_t n, void* out, si_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SHADOWINFER_HIP_H */
