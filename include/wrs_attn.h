/*
 * wrs_attn.h -- C ABI of the MI355X (gfx950) attention path for whisper.rs.
 *
 * Drop-in replacement for the reference's Flash-Attention-2 path
 * (crates/tensor/src/ops/attention.rs, crates/tensor/src/ops/softmax.rs,
 * crates/whisper/src/decoder.rs:131-264 and :835-892). Every entry point
 * returns an int status: 0 on success, a negative WRS_E* code otherwise, and
 * never unwinds across the ABI. Where the reference panics on a shape
 * assertion, the call returns WRS_EINVAL without touching any output; the
 * feature crate maps that back to a panic so the reference contract holds.
 *
 * Threading: a wrs_attn_ctx owns one HIP stream and its scratch memory and is
 * used by one thread at a time (one per WhisperState, like the reference's
 * per-state workspaces); independent contexts may run concurrently.
 * Host-slice entry points are synchronous. Device-resident entry points are
 * asynchronous on the context's stream.
 */
#ifndef WRS_ATTN_H
#define WRS_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define WRS_OK 0
#define WRS_EINVAL (-1)      /* shape/argument violation (reference: assert! panic) */
#define WRS_ENOMEM (-2)      /* device or host allocation failed */
#define WRS_EHIP (-3)        /* HIP runtime error; see wrs_attn_last_error */
#define WRS_EUNSUPPORTED (-4) /* valid for the reference, not handled on the GPU */
#define WRS_ERANGE (-5)      /* layer/slot index or length outside the arena */
#define WRS_ECAPTURE (-6)    /* context scratch would grow while the stream records a graph */
#define WRS_EBUSY (-7)       /* every slot of the GPU's fixed scratch is held by other contexts */

/* Element types of device-resident tensors. */
#define WRS_F32 0
#define WRS_F16 1
#define WRS_BF16 2

typedef struct wrs_attn_ctx wrs_attn_ctx;
typedef struct wrs_kv wrs_kv;

/* Strides, in elements, of a [batch][head][token][d] view of a tensor.
 * The reference's token-major rows [t][d_model] are
 * {batch: T*d_model, head: d_head, row: d_model}; a fused QKV projection
 * output [t][3*d_model] is the same with row = 3*d_model. */
typedef struct wrs_layout {
    int64_t batch_stride;
    int64_t head_stride;
    int64_t row_stride;
} wrs_layout;

/* ---- lifecycle ---------------------------------------------------------
 * No reference counterpart: the reference computes on host threads. The
 * context is what WhisperState would hold when whisper_context_params.use_gpu
 * / gpu_device (include/whisper.h:126-129) select this backend. */
int wrs_attn_create(int device, wrs_attn_ctx **out);
void wrs_attn_destroy(wrs_attn_ctx *ctx);
/* Queue work on a caller-owned hipStream_t; NULL is the device's null
 * (default) stream. A new context starts on a stream of its own. The switch
 * drains the previous stream (unless either stream records a graph), so the
 * previous stream must still exist: before destroying a stream the context
 * uses, switch the context to another stream or to NULL. */
int wrs_attn_set_stream(wrs_attn_ctx *ctx, void *hip_stream);
void *wrs_attn_get_stream(wrs_attn_ctx *ctx);
int wrs_attn_synchronize(wrs_attn_ctx *ctx);
/* Work decomposition of this context's prefill calls (wrs_attn_prefill, the
 * host-slice drop-ins and the prompt-row entry points); results do not depend
 * on it beyond floating-point summation order. No reference counterpart: the
 * reference's tiling is fixed (Q_TILE = KV_TILE = 128, attention.rs:13,26).
 * prefill_queries: queries per workgroup of the f16/bf16 kernel: 256 or 128
 * (four waves), -256, -192 or -128 for that many queries on eight, twelve or
 * eight waves whose halves take alternate 64-key tiles (key halves), -2 or -3
 * for 128-query blocks on that many such workgroups each (merged through
 * context scratch, allocated at the first such call), 32 for the key split (four
 * waves share a 32-query block's keys), or 0 to choose by grid size (the
 * default). f32_split: -1 chooses by
 * grid size (the default), 0 runs 128-query blocks, 1 the four-wave key
 * split, 2..4 the key split over that many waves, 5 the four-wave key split
 * with each block over several workgroups (merged through the same context
 * buffer). Other values: WRS_EINVAL. */
int wrs_attn_set_schedule(wrs_attn_ctx *ctx, int prefill_queries, int f32_split);
/* Text of the last error on this context (valid until the next call). */
const char *wrs_attn_last_error(wrs_attn_ctx *ctx);
const char *wrs_attn_status_string(int status);

/* Largest calls the context will serve, so that its scratch (split-K
 * partials, capture statistics, split f32 projection rows) is allocated now
 * rather than on the first call that needs it. No reference counterpart (the
 * reference allocates per call on the host). Device-resident entry points
 * never allocate once their sizes are reserved; a call that would grow
 * scratch while the context's stream records a graph fails with
 * WRS_ECAPTURE instead. One exception needs no reservation:
 * 16-bit prefill grids of fewer 128-query blocks than half the CUs merge
 * blocks split over two workgroups through a fixed context buffer (~9 MB on
 * 256 CUs), allocated by the first such call outside capture; during capture
 * before then, the call takes another schedule instead. Switching streams
 * (wrs_attn_set_stream) drains the old stream unless either stream is
 * recording a graph. Zero fields are ignored; reserving never shrinks.
 * Synchronous. */
typedef struct wrs_reserve {
    size_t n_heads;        /* heads of the planes decode and capture read */
    size_t decode_rows;    /* query rows of one decode call: slots or beams */
    size_t decode_keys;    /* longest cache one decode call reads */
    size_t capture_tokens; /* query rows of one alignment-head capture */
    size_t capture_keys;   /* n_audio of the captured cross plane */
    size_t linear_tokens;  /* rows of one f32-input projection (above 8) */
    size_t linear_n_in;    /* its input width */
} wrs_reserve;
int wrs_attn_reserve(wrs_attn_ctx *ctx, const wrs_reserve *r);

/* ---- host-slice drop-ins (synchronous; f32 host buffers) ---------------
 * Same arguments, argument meaning and results as the reference functions,
 * with slice lengths passed explicitly so the reference's length assertions
 * can be checked. */

/* pub fn flash_attention_2(q,k,v, t_q, t_kv, n_heads, d_model, causal, output)
 * crates/tensor/src/ops/attention.rs:68-78 (asserts :79-88). */
int wrs_flash_attention_2(wrs_attn_ctx *ctx, const float *q, size_t q_len, const float *k,
                          size_t k_len, const float *v, size_t v_len, size_t t_q, size_t t_kv,
                          size_t n_heads, size_t d_model, int causal, float *output,
                          size_t output_len);

/* pub fn multi_head_attention(...) -- same signature,
 * crates/tensor/src/ops/attention.rs:29-41. */
int wrs_multi_head_attention(wrs_attn_ctx *ctx, const float *q, size_t q_len, const float *k,
                             size_t k_len, const float *v, size_t v_len, size_t t_q, size_t t_kv,
                             size_t n_heads, size_t d_model, int causal, float *output,
                             size_t output_len);

/* pub fn single_token_mha_d64(q,k,v, t_kv, n_heads, d_model, output)
 * crates/tensor/src/ops/attention.rs:246-254. */
int wrs_single_token_mha_d64(wrs_attn_ctx *ctx, const float *q, size_t q_len, const float *k,
                             size_t k_len, const float *v, size_t v_len, size_t t_kv,
                             size_t n_heads, size_t d_model, float *output, size_t output_len);

/* fn multi_head_attention_with_cache(q,k,v, n_tokens, total_tokens, t_past,
 * n_heads, d_model, output) -- crates/whisper/src/decoder.rs:835-892
 * (private in the reference; exported so the decoder can route through it). */
int wrs_mha_with_cache(wrs_attn_ctx *ctx, const float *q, size_t q_len, const float *k,
                       size_t k_len, const float *v, size_t v_len, size_t n_tokens,
                       size_t total_tokens, size_t t_past, size_t n_heads, size_t d_model,
                       float *output, size_t output_len);

/* ---- device-resident prefill (asynchronous) ----------------------------
 * flash_attention_2 (crates/tensor/src/ops/attention.rs:68-243) over `batch`
 * independent windows, called from crates/whisper/src/encoder.rs:289-299.
 * q/k/v/out are device pointers; out is f32. Queries are causal-masked
 * against keys j <= i + q_pos_offset when `causal` is set (q_pos_offset = 0
 * is the reference's mask; t_past is the decoder prompt's,
 * crates/whisper/src/decoder.rs:861). Supported types: q_dtype == kv_dtype
 * in {F16, BF16} (d_head 64 runs on the 16-bit MFMA kernel, other d_head on
 * the f32 one), and q F32 with kv F32/F16/BF16 (f32 accumulate-check kernel).
 * d_head <= 128. 16-bit tensors need 16-byte aligned rows (strides multiple
 * of 8 elements). The 16-bit kernel forms the PV product in f16: for bf16
 * inputs, a workgroup whose outputs come out inf/NaN (a V value of magnitude
 * >= 65536) recomputes its queries with f32 operands in the same launch, so
 * any finite bf16 input gives a finite, f32-accurate result. Grids of fewer
 * 128-query blocks than half the CUs over long key ranges (one whisper-tiny
 * or -base window) merge split blocks through a context buffer that the first
 * such call outside stream capture allocates (wrs_attn_reserve). */
int wrs_attn_prefill(wrs_attn_ctx *ctx, int q_dtype, const void *q, const wrs_layout *q_layout,
                     int kv_dtype, const void *k, const wrs_layout *k_layout, const void *v,
                     const wrs_layout *v_layout, float *out, const wrs_layout *out_layout,
                     size_t batch, size_t n_heads, size_t t_q, size_t t_kv, size_t d_head,
                     int causal, size_t q_pos_offset);

/* ---- device KV arena ---------------------------------------------------
 * pub struct DecoderKvCache (crates/whisper/src/decoder.rs:131-145), in HBM:
 * self K/V [layer][slot][head][max_ctx][64], cross K/V
 * [layer][head][n_audio_max][64]; d_head is 64, d_model = n_heads*64.
 * Slot lengths (the reference's t_past vector) are kept on the host.
 * Planes are f16 (wrs_kv_create: the MFMA and split-K decode kernels) or f32
 * (wrs_kv_create_dtype with WRS_F32: the reference's own f32 cache, twice the
 * bytes, with the reference's arithmetic -- decode, cached prompt rows and
 * single cross rows on the exact decode kernel, as the host-slice
 * single_token_mha_d64 / mha_with_cache run; cross prompt rows on the f32
 * prefill kernel, as wrs_flash_attention_2 runs them; capture with f32
 * scores). On f32 arenas wrs_attn_decode_cross_noalloc,
 * wrs_attn_prefill_cross_lse and wrs_attn_capture_cross_heads_lse return
 * WRS_EUNSUPPORTED, and the attention calls size their score scratch
 * (rows x heads x keys floats) on the first call, so a first call under
 * stream capture fails with WRS_ECAPTURE. */

/* DecoderKvCache::new (decoder.rs:148-157) with the arena capacity fixed;
 * f16 planes. */
int wrs_kv_create(wrs_attn_ctx *ctx, size_t n_layers, size_t n_slots, size_t n_heads,
                  size_t max_ctx, size_t n_audio_max, wrs_kv **out);
/* The same with the plane element type: WRS_F16 or WRS_F32 (the reference
 * cache's Vec<f32>, decoder.rs:131-157). */
int wrs_kv_create_dtype(wrs_attn_ctx *ctx, size_t n_layers, size_t n_slots, size_t n_heads,
                        size_t max_ctx, size_t n_audio_max, int dtype, wrs_kv **out);
/* Plane element type of an arena (WRS_F16 or WRS_F32). No reference
 * counterpart: the reference cache has one type. */
int wrs_kv_dtype(wrs_kv *kv, int *dtype);
void wrs_kv_destroy(wrs_kv *kv);
/* DecoderKvCache::clear (decoder.rs:162-176): every slot length to 0. */
int wrs_kv_clear(wrs_kv *kv);
/* DecoderKvCache::clear_slot (decoder.rs:179-189). */
int wrs_kv_clear_slot(wrs_kv *kv, size_t slot);
/* DecoderKvCache::invalidate_cross (decoder.rs:196-203). */
int wrs_kv_invalidate_cross(wrs_kv *kv);
/* DecoderKvCache::ensure_slots (decoder.rs:207-218): grows, keeps contents. */
int wrs_kv_ensure_slots(wrs_kv *kv, size_t n_slots);
/* DecoderKvCache::copy_slot (decoder.rs:223-236): valid prefix of src -> dst. */
int wrs_kv_copy_slot(wrs_kv *kv, size_t dst, size_t src);
/* DecoderKvCache::slot_len (decoder.rs:239-241). */
int wrs_kv_slot_len(wrs_kv *kv, size_t slot, size_t *len);
/* `cache.t_past[slot] = n_past` rewind (crates/ffi/src/lib.rs:2352 with the
 * truncation at decoder.rs:626-630); len must not exceed the stored rows. */
int wrs_kv_set_len(wrs_kv *kv, size_t slot, size_t len);
/* DecoderKvCache::slide_to_fit (decoder.rs:248-263); *pos gets t_past. */
int wrs_kv_slide_to_fit(wrs_kv *kv, size_t slot, size_t n_new, size_t max_ctx, size_t *pos);
/* Append of decoder.rs:631-635: write n rows (f32 [n][d_model]) of this
 * layer's K and V at the slot's current length; lengths advance only with
 * wrs_kv_advance, after all layers (decoder.rs:765-767). src_on_host selects
 * host or device source pointers. */
int wrs_kv_append(wrs_kv *kv, size_t layer, size_t slot, const float *k_rows,
                  const float *v_rows, size_t n, int src_on_host);
int wrs_kv_advance(wrs_kv *kv, size_t slot, size_t n);
/* Store of precompute_cross_attn (decoder.rs:423-447): f32 [n_audio][d_model]
 * K and V of one layer, into the head planes (converted to f16, or copied). */
int wrs_kv_set_cross(wrs_kv *kv, size_t layer, const float *k, const float *v, size_t n_audio,
                     int src_on_host);
/* n_audio of one layer's stored cross K/V (DecoderKvCache keeps cross K/V per
 * layer, decoder.rs:136-139); 0 after wrs_kv_invalidate_cross. */
int wrs_kv_cross_len(wrs_kv *kv, size_t layer, size_t *n_audio);
/* Raw device pointers of the arena planes (for tests and fused callers);
 * elements are of the arena's dtype, the slot stride in elements. */
int wrs_kv_self_planes(wrs_kv *kv, void **k, void **v, size_t *slot_stride_elems);
int wrs_kv_cross_planes(wrs_kv *kv, void **k, void **v);

/* ---- device-resident decode (asynchronous) -----------------------------
 * Self-attention step: decoder.rs:613-647 -> multi_head_attention_with_cache
 * -> single_token_mha_d64 (decoder.rs:852-855) for every slot in one launch.
 * Row i of q ([n][d_model] f32, device) belongs to slots[i] (host array) and
 * sits at position slot_len(slots[i]); its K/V row must already be appended,
 * so it attends slot_len + 1 keys. out: [n][d_model] f32 device. */
int wrs_attn_decode_self(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, const size_t *slots,
                         size_t n, const float *q, float *out);
/* Cross-attention step: decoder.rs:689-724 -> multi_head_attention ->
 * single_token_mha_d64 (attention.rs:102-105), all n_beams query rows of one
 * utterance against the shared cross plane in one launch (K/V read once).
 * A layer without cross K/V (never set, invalidated, or an arena created with
 * n_audio_max = 0) gives zero rows, as t_kv == 0 does (attention.rs:93-96). */
int wrs_attn_decode_cross(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, const float *q,
                          size_t n_beams, float *out); /* q 16-byte aligned */
/* Allocation-free variant of wrs_attn_decode_cross, with the same arguments
 * and results. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Its split-K partials and merge counters
 * live in a fixed device array of the library (4 slots of 512 KiB + 16 KiB,
 * one array per GPU, held until the process ends), so it never calls
 * hipMalloc or hipFree. A context claims one slot of its GPU on its first
 * call here and releases it in wrs_attn_destroy; with all four held by other
 * live contexts the call fails with WRS_EBUSY. Limits per call: at most 128
 * heads, and for n_audio above 256 (shorter planes need no partials)
 * min(n_beams, 8) x n_heads x ceil(n_audio / 128) x 68 <= 131072 floats
 * (large-v3: up to 8 beams); larger shapes fail with WRS_ERANGE. q must be
 * 16-byte aligned (WRS_EINVAL otherwise). Calls of one context are ordered on
 * its stream; two contexts never share a slot. */
int wrs_attn_decode_cross_noalloc(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, const float *q,
                                  size_t n_beams, float *out);
/* Multi-token rows (prompt prefill): decoder.rs:857-891 self-attention with
 * offset t_past = slot_len(slot) over the slot's f16 cache (rows appended),
 * and attention.rs:107-243 cross-attention with t_q = n_tokens (the rows run
 * on the split-K decode kernel in groups of 8 that share each read of the
 * plane, with its numerics: f16 keys and values, q split into two f16 parts). */
int wrs_attn_prefill_self(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, size_t slot,
                          const float *q, size_t n_tokens, float *out);
int wrs_attn_prefill_cross(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, const float *q,
                           size_t n_tokens, float *out); /* q 16-byte aligned */
/* wrs_attn_prefill_cross (the multi_head_attention call of decoder.rs:698-708)
 * that also writes each row's softmax statistics for
 * wrs_attn_capture_cross_heads_lse: lse is an f32
 * device buffer of n_heads * n_tokens * 2 values, (max, sum) of row i of head
 * h at 2 * (h * n_tokens + i), in the exp2 domain: max = log2(e) * max_j s_ij,
 * sum = sum_j exp2(log2(e) * s_ij - max), s_ij = q_i.k_j / 8. Not written when
 * the layer has no cross keys. */
int wrs_attn_prefill_cross_lse(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, const float *q,
                               size_t n_tokens, float *out, float *lse); /* q 16-byte aligned */

/* ---- alignment-head capture (asynchronous) -----------------------------
 * fn capture_cross_attention_heads(q, k, n_tokens, n_audio, n_heads, d_model,
 * selected, n_selected, row_offset, out, scores) -- decoder.rs:796-828, as
 * called per text layer from decoder.rs:709-721. k is this layer's cross
 * plane of the arena (n_audio = wrs_kv_cross_len); selected is given as two
 * host arrays, pair p = (slots[p], heads[p]). q: [n_tokens][d_model] f32
 * device, 16-byte aligned; out: f32 device buffer of out_len elements,
 * written at [(row_offset + i) * n_selected + slots[p]][0..n_audio). The
 * reference's scores scratch is internal (chunk statistics in the context). */
int wrs_attn_capture_cross_heads(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer, const float *q,
                                 size_t n_tokens, const size_t *slots, const size_t *heads,
                                 size_t n_pairs, size_t n_selected, size_t row_offset,
                                 float *out, size_t out_len);
/* The same capture in one launch, for the decoder's order of calls
 * (decoder.rs:698-721: the cross-attention of the same q rows runs first):
 * lse is what wrs_attn_prefill_cross_lse wrote for these q rows and this
 * layer, and the weights are exp2(log2(e) * s - max) / sum with them. The
 * statistics come from the attention kernel's own score sums, whose rounding
 * differs from this kernel's exact-product sums: weights agree with
 * wrs_attn_capture_cross_heads to ~1e-6 relative, rows sum to 1 within 1e-5. */
int wrs_attn_capture_cross_heads_lse(wrs_attn_ctx *ctx, wrs_kv *kv, size_t layer,
                                     const float *q, size_t n_tokens, const size_t *slots,
                                     const size_t *heads, size_t n_pairs, size_t n_selected,
                                     size_t row_offset, float *out, size_t out_len,
                                     const float *lse);

/* ---- projections with f16 weights (asynchronous) -----------------------
 * LinearWeight::linear with F16 weights (crates/tensor/src/weight.rs:116-137
 * -> crates/tensor/src/ops/quant.rs:415-473 f16_linear):
 * out(t, r) = W[r] . x[t] + bias[r], W [n_out][n_in] f16 row-major (the ggml
 * halves), bias f32 or NULL, x [n_tokens] rows of n_in (row stride in
 * elements) as f32 (split into two f16 parts: products to 2^-22) or f16. x_len and out_len are the
 * buffers' lengths in elements, checked like the reference's length asserts
 * (quant.rs:424-425). out(t, r) is written in
 * out_dtype at out + t*out_row_stride + (r/64)*out_head_stride + r%64:
 * out_head_stride = 64 gives the reference's token-major [t][n_out] rows
 * (encoder.rs:275-277's fused QKV output, read in place by wrs_attn_prefill).
 * All pointers are device pointers. n_in % 64 == 0. Batches of up to 8 rows
 * (the beams of a decode step, f16_gemv_parallel at quant.rs:392-413) run on
 * the weight-stream kernel and take any n_out; larger ones need n_out % 4 == 0. */
int wrs_linear(wrs_attn_ctx *ctx, int x_dtype, const void *x, size_t x_len,
               int64_t x_row_stride, const void *w, const float *bias, size_t n_tokens,
               size_t n_in, size_t n_out, int out_dtype, void *out, size_t out_len,
               int64_t out_row_stride, int64_t out_head_stride);

/* Several projections of one input in one launch (replaces the consecutive
 * LinearWeight::linear calls on one normalized input at
 * crates/whisper/src/decoder.rs:597-611: self-attention q, k and v). Group g
 * computes out[g](t, r) = w[g][r] . x[t] + bias[g][r] exactly as wrs_linear
 * does; all groups share x, n_out and the output layout. bias may be NULL, or
 * hold NULL entries; out_len[g] is out[g]'s length in elements.
 * n_groups <= 64. */
int wrs_linear_group(wrs_attn_ctx *ctx, int x_dtype, const void *x, size_t x_len,
                     int64_t x_row_stride, size_t n_groups, const void *const *w,
                     const float *const *bias, size_t n_tokens, size_t n_in, size_t n_out,
                     int out_dtype, void *const *out, const size_t *out_len,
                     int64_t out_row_stride, int64_t out_head_stride);

/* Activations for wrs_linear_fused. */
#define WRS_ACT_NONE 0
#define WRS_ACT_GELU 1 /* crates/tensor/src/ops/gelu.rs:11-23, applied in f32 */

/* layer_norm -> linear (one or more weight groups) -> optional GELU, as one
 * launch for decode-sized batches (replaces, at crates/whisper/src/decoder.rs,
 * the layer_norm of :586-594 with the q/k/v linears of :597-611, that of
 * :660-668 with the cross-attention q linear, and that of :737-745 with mlp0
 * and the gelu_inplace of :753). The values equal wrs_layer_norm (f32 out) on
 * x, then wrs_linear_group on the normalized rows, then wrs_gelu_inplace on
 * each output (before rounding when out_dtype is f16/bf16). x is f32;
 * ln_gamma and ln_beta (16-byte aligned, n_in values) are both NULL to skip
 * the norm; activation is WRS_ACT_NONE or WRS_ACT_GELU. Batches above 8 rows
 * (or x beyond the weight-stream kernel's LDS) run the norm as its own
 * launch and then need packed rows (x_row_stride == n_in). */
int wrs_linear_fused(wrs_attn_ctx *ctx, const float *x, size_t x_len, int64_t x_row_stride,
                     const float *ln_gamma, const float *ln_beta, float ln_eps,
                     size_t n_groups, const void *const *w, const float *const *bias,
                     size_t n_tokens, size_t n_in, size_t n_out, int activation,
                     int out_dtype, void *const *out, const size_t *out_len,
                     int64_t out_row_stride, int64_t out_head_stride);

/* pub fn layer_norm(input, gamma, beta, eps, num_tokens, d_model, output)
 * -- crates/tensor/src/ops/norm.rs:116-143 (asserts :124-127), device f32 rows;
 * the output may be rounded to f16 / bf16 for a following projection.
 * d_model % 4 == 0. */
int wrs_layer_norm(wrs_attn_ctx *ctx, const float *x, size_t x_len, const float *gamma,
                   const float *beta, float eps, size_t n_tokens, size_t d_model, int out_dtype,
                   void *out, size_t out_len);
/* pub fn gelu_inplace(data) -- crates/tensor/src/ops/gelu.rs:11-23, tanh form,
 * in place on device f32. */
int wrs_gelu_inplace(wrs_attn_ctx *ctx, float *data, size_t n);

/* WhisperDecoder::precompute_cross_attn (crates/whisper/src/decoder.rs:423-447)
 * straight into the arena: for every layer l, K = enc . w_k[l]^T and
 * V = enc . w_v[l]^T + b_v[l] (b_v may be NULL, or hold NULL entries), stored
 * as the f16 cross planes; every layer's cross length becomes n_audio. enc is
 * [n_audio] rows of d_model (f32 or f16, device); w_k / w_v / b_v are host
 * arrays of n_layers device pointers. */
int wrs_kv_set_cross_proj(wrs_kv *kv, int x_dtype, const void *enc, size_t enc_len,
                          int64_t enc_row_stride, size_t n_audio, const void *const *w_k,
                          const void *const *w_v, const float *const *b_v);

/* ---- measurement helper ----------------------------------------------------
 * No reference counterpart: reads `bytes` of device memory (16-byte aligned,
 * a multiple of 16) once, in one launch shaped like the split-K decode's grid
 * (512 threads x 64 bytes per workgroup), and writes one float per workgroup
 * to sink (sink_len >= ceil(bytes / 32768)). It measures the practical floor
 * of a decode-sized launch (launch, ramp and DRAM latency included).
 * Asynchronous. */
int wrs_stream_read(wrs_attn_ctx *ctx, const void *src, size_t bytes, float *sink,
                    size_t sink_len);
/* The same read with another launch shape: `threads` per workgroup (256,
 * 512 or 1024) and `loads_per_lane` 16-byte loads per lane (1, 2, 4, 8, 16
 * or 24), all issued before any is used; sink_len >= ceil(bytes /
 * (16 * threads * loads_per_lane)). Other shapes: WRS_EINVAL. Asynchronous. */
int wrs_stream_read_shape(wrs_attn_ctx *ctx, const void *src, size_t bytes, int threads,
                          int loads_per_lane, float *sink, size_t sink_len);

#ifdef __cplusplus
}
#endif
#endif /* WRS_ATTN_H */
