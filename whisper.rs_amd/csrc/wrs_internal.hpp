// Internal declarations shared by the HIP kernels and the C-ABI runtime.
//
// Layout conventions (all strides in elements, not bytes):
//   activations  element (b, h, t, d) at base + b*bs + h*hs + t*rs + d
//                (token-major [T][n_heads*d_head] rows of the reference are
//                 hs = d_head, rs = d_model; BHSD is hs = T*d_head, rs = d_head)
//   KV cache     f16 (or f32), one [ctx][64] plane per (layer, slot, head) --
//                rows of one head are contiguous 128-byte (256-byte) lines.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wrs {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// Activation applied by a projection's epilogue, in f32 before the output
// rounding (the reference runs gelu_inplace on the f32 projection output).
enum Act : int { kActNone = 0, kActGelu = 1 };

// GELU, tanh form, in the reference's order of operations with contraction
// off (crates/tensor/src/ops/gelu.rs:6-23; constants gelu.rs:3-4).
__device__ inline float gelu_tanh(float x) {
#pragma clang fp contract(off)
  const float kA = 0.044715f, kS = 0.7978846f;
  const float inner = kS * x * (1.0f + kA * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

struct Layout {
  int64_t bs;  // batch (window) stride
  int64_t hs;  // head stride
  int64_t rs;  // row (token) stride
};

// Logical workgroup id with an XCD-aware remap: the hardware hands linear ids
// round-robin to the 8 XCDs, so consecutive logical ids (the query blocks of
// one (window, head), which read the same K/V) are gathered onto one XCD and
// share its L2.
__device__ inline int xcd_remap(int pid, int nwg) {
  const int xcd = pid & 7, k = pid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
}

// Agent-scope (L2-coherent across the GPU's XCDs) store and load of one
// float, for partials that another workgroup of the launch merges.
__device__ inline void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Flash-attention prefill over full query/key sequences
// (crates/tensor/src/ops/attention.rs:68-243 semantics).
struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  float* o;
  Layout lq, lk, lv, lo;
  int batch, n_heads, t_q, t_kv, d_head;
  int causal;        // mask keys j > i + q_pos_offset
  int q_pos_offset;  // absolute position of query row 0 (decoder prompt: t_past)
  float scale;       // 1/sqrt(d_head), rounded to f32 like attention.rs:107
  // Schedule overrides from the context (wrs_attn_set_schedule): queries per
  // workgroup of the 16-bit kernel (0 = by grid size), and the f32 kernel's
  // key split (-1 = by grid size, 0 = 128-query blocks, 1 = four waves,
  // 2..4 = that many waves, 5 = four waves over several workgroups).
  int force_queries;
  int force_f32_split;
  // Context scratch for grids whose blocks split their keys over several
  // workgroups (null when none is available): partials and merge counters
  // (zero between launches), with their sizes.
  float* split_part;
  size_t split_part_floats;
  unsigned* split_counters;
  size_t split_counter_words;
};

// MFMA f16/bf16 kernel, d_head == 64, q/k/v of one 16-bit type, rows 16-byte
// aligned; prefill_mfma16_supports() states the remaining shape limits.
bool prefill_mfma16_supports(const PrefillArgs& a);
// Scratch the 16-bit kernel's schedule for `a` uses (floats of partials and
// words of counters), both 0 when it uses none.
void prefill_mfma16_scratch(const PrefillArgs& a, size_t* part_floats, size_t* counter_words);
// The sizes the context allocates at least: enough for every grid whose
// blocks the default schedule splits over workgroups.
size_t prefill_split_floats_min();
size_t prefill_split_words_min();
hipError_t launch_prefill_mfma16(const PrefillArgs& a, DType dt, hipStream_t s);
// f32-accumulate-check kernel on f32 MFMA: q f32, k/v f32|f16|bf16 widened
// exactly to f32, any d_head <= 128.
hipError_t launch_prefill_f32(const PrefillArgs& a, DType q_dt, DType kv_dt, hipStream_t s);
// Scratch its schedule for `a` uses (as prefill_mfma16_scratch).
void prefill_f32_scratch(const PrefillArgs& a, size_t* part_floats, size_t* counter_words);

// Exact reference decode semantics on f32 K/V (attention.rs:246-434
// single_token_mha_d64 and decoder.rs:835-892): full score row, softmax with
// reciprocal multiply, weights < 1e-7 skipped. Rows come in groups of
// rows_per_group that share one K/V base (goff[g] elements past k and v);
// row i of group g sees keys [0, glen[g] + i * limit_step). Host slices are
// one group of token-major rows (kv_rs = d_model, kv_hs = d_head); the f32
// arena passes [head][ctx][64] planes (kv_rs = 64, kv_hs = the plane).
constexpr int kMaxExactGroups = 64;
struct ExactArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_rs, o_rs;   // row strides of q and out (head h at h * d_head)
  int64_t kv_rs, kv_hs;  // K/V: key row and head strides
  int n_rows, n_heads, d_head;
  int rows_per_group, n_groups, limit_step;
  float scale;
  float* scores;  // scratch [n_rows][n_heads][scores_stride]
  int64_t scores_stride;
  int64_t goff[kMaxExactGroups];
  int glen[kMaxExactGroups];
};
hipError_t launch_decode_exact_f32(const ExactArgs& a, hipStream_t s);

// Split-K decode over an f16 KV cache: one query row per (group, row),
// all rows of a group share one K/V plane set (cross-attention: the beams of
// one utterance; self-attention: one row per slot).
constexpr int kMaxDecodeGroups = 64;
constexpr int kMaxRowsPerGroup = 8;
struct DecodeArgs {
  const float* q;   // row (g*rows_per_group + r): q + row*q_rs + h*64
  float* o;         // same indexing with o_rs
  const _Float16* k;  // plane (g, h): k + goff[g] + h*kv_hs, key j at +j*64
  const _Float16* v;
  int64_t q_rs, o_rs, kv_hs;
  int64_t goff[kMaxDecodeGroups];  // per-group plane offset (elements)
  int len[kMaxDecodeGroups];       // keys visible to group g
  int n_groups, rows_per_group, n_heads;
  int chunk;     // keys per workgroup (kDecodeChunk or kDecodeChunkLong)
  int n_splits;  // workgroups per (group, head) = ceil(max len / chunk)
  float scale_log2;  // (1/8) * log2(e)
  float* part;        // scratch: [groups][heads][splits][rows][68]
  unsigned* counters;  // scratch: one per (group, head) every 32 words, zero between launches
  // Optional: row statistics (max, sum of exp2(s - max)) of output row
  // lse_row0 + g*rows_per_group + r for head h at lse[2 * (h * lse_rows + row)].
  float* lse;
  int lse_rows, lse_row0;
};
constexpr int kDecodeChunk = 128;
constexpr int kDecodeChunkLong = 256;  // one workgroup per (group, head) up to this length
hipError_t launch_decode_f16(const DecodeArgs& a, hipStream_t s);
size_t decode_part_floats(int n_groups, int n_heads, int n_splits, int rows);
size_t decode_counter_words(int n_groups, int n_heads);

// Measurement: a streaming read of `bytes` (multiple of 16, 16-byte aligned)
// with the split-K decode's grid shape (512 threads x 64 bytes per
// workgroup); sink receives stream_read_blocks(bytes) floats.
hipError_t launch_stream_read(const void* src, int64_t bytes, float* sink, hipStream_t s);
int64_t stream_read_blocks(int64_t bytes);
// The same with `threads` per workgroup (256, 512, 1024) and `loads` 16-byte
// loads per lane (1, 2, 4, 8, 16, 24).
hipError_t launch_stream_read_shape(const void* src, int64_t bytes, int threads, int loads,
                                    float* sink, hipStream_t s);
int64_t stream_read_shape_blocks(int64_t bytes, int threads, int loads);

// Alignment-head capture over the f16 cross plane
// (decoder.rs:796-828 semantics): for query row i and pair p,
// softmax_j(dot(q_i[head_p], k_j[head_p]) * scale) into
// out[((row_offset + i) * n_selected + slot_p) * n_audio + j].
constexpr int kCaptureRows = 16;       // query rows per workgroup
constexpr int kCaptureChunk = 128;     // keys per workgroup
constexpr int kMaxCapturePairs = 32;   // (slot, head) pairs per launch
struct CaptureArgs {
  const float* q;     // row i, head h: q + i*q_rs + h*64
  const _Float16* k;  // plane of head h: k + h*kv_hs, key j at +j*64
  const float* k32;   // the same for f32 planes (capture_cross_f32)
  float scale;        // 1/sqrt(64), capture_cross_f32
  float* out;
  float* part;        // scratch: capture_part_floats(n_pairs, n_tokens, n_audio)
  int64_t q_rs, kv_hs;
  int n_tokens, n_audio, n_selected, row_offset, n_pairs;
  float scale_log2;  // log2(e)/sqrt(64): decoder.rs:810's scale in the exp2 domain
  // When set: per-row softmax statistics of the attention pass over the same q
  // and keys, (max, sum) in the exp2 domain at lse[2 * (head * n_tokens + row)];
  // the capture then runs as one pass.
  const float* lse;
  int slot[kMaxCapturePairs];
  int head[kMaxCapturePairs];
};
size_t capture_part_floats(int n_pairs, int n_tokens, int n_audio);
hipError_t launch_capture_cross_f16(const CaptureArgs& a, hipStream_t s);
// Over f32 planes (k32, scale; no part, no lse): one workgroup per (row, pair).
hipError_t launch_capture_cross_f32(const CaptureArgs& a, hipStream_t s);

// Projections with f16 weights (quant.rs:415-473 semantics):
// out(t, r) = row_scale[t] * (W[r] . x'[t]) + bias[r] with W [n_out][n_in] f16
// and x' [n_tokens][k_total] f16 (k_total = n_in, or kSplitParts n_in for split
// f32 rows, whose weight column is k' mod n_in). Element (t, r) is stored at
// out + t*out_rs + (r/64)*out_hs + r%64. Groups share x and differ in W, bias
// and out (all layers' cross K and V in one launch).
constexpr int kLinearK = 64;          // n_in must be a multiple of this
constexpr int kSplitParts = 2;        // f16 parts of a split f32 row: hi, lo
constexpr int kMaxLinearGroups = 64;
struct LinearArgs {
  const _Float16* x;
  int64_t x_rs;
  const float* row_scale;  // nullable: 1
  int n_tokens, n_in, n_out, k_total, n_groups;
  int64_t out_rs, out_hs;
  int act;  // Act, applied after the bias
  const _Float16* w[kMaxLinearGroups];
  const float* bias[kMaxLinearGroups];  // nullable entries
  void* out[kMaxLinearGroups];
};
hipError_t launch_linear_f16w(const LinearArgs& a, DType out_dt, hipStream_t s);
// Decode-sized batches (n_tokens <= kGemvMaxRows) of the same product on the
// f16 weight stream; x is f32 or f16 with row stride x_rs, no split needed.
constexpr int kGemvMaxRows = 8;
constexpr int kGemvXFloats = 40960;  // n_tokens * n_in staged in LDS (160 KB)
struct GemvArgs {
  const void* x;
  int64_t x_rs;
  int n_tokens, n_in, n_out, n_groups;
  int64_t out_rs, out_hs;
  // Optional LayerNorm of every x row before the product (norm.rs:116-143,
  // the layer_norm_rows arithmetic exactly; f32 x only): ln_g null = none.
  const float* ln_g;
  const float* ln_b;
  float ln_eps;
  int act;  // Act, applied after the bias
  const _Float16* w[kMaxLinearGroups];
  const float* bias[kMaxLinearGroups];
  void* out[kMaxLinearGroups];
};
hipError_t launch_gemv_f16w(const GemvArgs& a, DType x_dt, DType out_dt, hipStream_t s);
// f32 rows -> [hi | lo] f16 rows (kSplitParts n_in each) and per-row 2^-shift.
hipError_t launch_linear_split(const float* x, int64_t x_rs, int n_tokens, int n_in,
                               _Float16* xs, float* row_scale, hipStream_t s);

// LayerNorm over f32 rows (norm.rs:116-143), output f32/f16/bf16 rows of d;
// d % 4 == 0, rows 16-byte aligned.
hipError_t launch_layer_norm(const float* x, const float* gamma, const float* beta, float eps,
                             int n_tokens, int d, DType out_dt, void* out, hipStream_t s);
// GELU, tanh form, in place on f32 (gelu.rs:11-23); data 16-byte aligned.
hipError_t launch_gelu(float* data, int64_t n, hipStream_t s);

// Zero fills issued as kernels (never as memset nodes, so that a caller may
// capture them into a graph): f32 element (b, h, r, c) at
// base + b*bs + h*hs + r*rs + c for c < cols; and n 32-bit words.
hipError_t launch_fill_zero_rows(float* base, int64_t bs, int64_t hs, int64_t rs, int batch,
                                 int n_heads, int n_rows, int cols, hipStream_t s);
hipError_t launch_fill_zero_u32(unsigned* p, int64_t n, hipStream_t s);

// KV arena kernels.
// f32 rows [n][d_model] (row stride src_rs) -> f16 planes: head h, row i at
// dst + h*dst_hs + (pos + i)*64.
hipError_t launch_kv_write_rows(const float* src, int64_t src_rs, int n, int n_heads,
                                _Float16* dst, int64_t dst_hs, int pos, hipStream_t s);
// The same into f32 planes (a copy).
hipError_t launch_kv_write_rows_f32(const float* src, int64_t src_rs, int n, int n_heads,
                                    float* dst, int64_t dst_hs, int pos, hipStream_t s);
// Planes of one slot: plane (l, h) at base + l*layer_stride + h*plane_stride,
// in rows of 64 f16 (an f32 plane is passed as twice the rows and strides).
// Move rows [drop, len) of every plane down to [0, len - drop).
hipError_t launch_kv_slide(_Float16* base, int64_t layer_stride, int64_t plane_stride,
                           int n_layers, int n_heads, int len, int drop, hipStream_t s);
// Copy rows [0, len) of every plane from src to dst (same plane geometry).
hipError_t launch_kv_copy_planes(const _Float16* src, _Float16* dst, int64_t layer_stride,
                                 int64_t plane_stride, int n_layers, int n_heads, int len,
                                 hipStream_t s);

}  // namespace wrs
