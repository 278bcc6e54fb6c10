//! The Flash-Attention-2 path of `whisper-tensor` on an AMD Instinct MI355X
//! (gfx950), through the C ABI of `libwrs_attn` (`include/wrs_attn.h`).
//!
//! The crate lives outside the workspace's `crates/` tree and has no
//! dependencies, so the pure-Rust default build and its architecture gate
//! (`scripts/check_pure_rust.sh`, checks 3 and 4) are untouched. It is pulled
//! in only by `whisper-tensor`'s optional `hip` feature, whose entry points
//! forward here:
//!
//! * [`flash_attention_2`], [`multi_head_attention`] and
//!   [`single_token_mha_d64`] have the signatures of
//!   `crates/tensor/src/ops/attention.rs:29-41`, `:68-78` and `:246-254`;
//!   [`multi_head_attention_with_cache`] that of the decoder's private
//!   `crates/whisper/src/decoder.rs:835-845`. Each runs on the calling
//!   thread's own context (one HIP stream and scratch per thread, as the
//!   reference keeps one workspace per `WhisperState`), synchronously on host
//!   slices, with the reference's results and panics.
//! * [`set_device`] selects the GPU (the caller maps
//!   `whisper_context_params.use_gpu` / `gpu_device`, `include/whisper.h:126-129`,
//!   onto it); [`enabled`] is what the `cfg(feature = "hip")` branches test.
//! * [`ffi`] declares every C entry point, including the device-resident ones
//!   (batched prefill, the device KV arena, split-K decode, projections) that
//!   the fast integration level uses.
#![allow(clippy::too_many_arguments)]

use std::cell::RefCell;
use std::ffi::{c_int, c_void, CStr};
use std::sync::atomic::{AtomicI32, Ordering};

/// Raw declarations of `include/wrs_attn.h`, one per C entry point.
pub mod ffi {
    use std::ffi::{c_char, c_int, c_void};

    /// `wrs_attn_ctx`: one device, one stream, private scratch.
    #[repr(C)]
    pub struct WrsCtx {
        _p: [u8; 0],
    }
    /// `wrs_kv`: the device KV arena (`DecoderKvCache`, decoder.rs:131-264).
    #[repr(C)]
    pub struct WrsKv {
        _p: [u8; 0],
    }

    /// `wrs_layout`: element strides of a `[batch][head][token][d]` view.
    #[repr(C)]
    #[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
    pub struct WrsLayout {
        pub batch_stride: i64,
        pub head_stride: i64,
        pub row_stride: i64,
    }

    /// `wrs_reserve`: the largest calls a context serves.
    #[repr(C)]
    #[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
    pub struct WrsReserve {
        pub n_heads: usize,
        pub decode_rows: usize,
        pub decode_keys: usize,
        pub capture_tokens: usize,
        pub capture_keys: usize,
        pub linear_tokens: usize,
        pub linear_n_in: usize,
    }

    pub const WRS_OK: c_int = 0;
    pub const WRS_EINVAL: c_int = -1;
    pub const WRS_ENOMEM: c_int = -2;
    pub const WRS_EHIP: c_int = -3;
    pub const WRS_EUNSUPPORTED: c_int = -4;
    pub const WRS_ERANGE: c_int = -5;
    pub const WRS_ECAPTURE: c_int = -6;
    pub const WRS_EBUSY: c_int = -7;

    pub const WRS_F32: c_int = 0;
    pub const WRS_F16: c_int = 1;
    pub const WRS_BF16: c_int = 2;

    pub const WRS_ACT_NONE: c_int = 0;
    pub const WRS_ACT_GELU: c_int = 1;

    extern "C" {
        // lifecycle (no reference counterpart)
        pub fn wrs_attn_create(device: c_int, out: *mut *mut WrsCtx) -> c_int;
        pub fn wrs_attn_destroy(ctx: *mut WrsCtx);
        pub fn wrs_attn_set_stream(ctx: *mut WrsCtx, hip_stream: *mut c_void) -> c_int;
        pub fn wrs_attn_get_stream(ctx: *mut WrsCtx) -> *mut c_void;
        pub fn wrs_attn_set_schedule(
            ctx: *mut WrsCtx,
            prefill_queries: c_int,
            f32_split: c_int,
        ) -> c_int;
        pub fn wrs_attn_synchronize(ctx: *mut WrsCtx) -> c_int;
        pub fn wrs_attn_last_error(ctx: *mut WrsCtx) -> *const c_char;
        pub fn wrs_attn_status_string(status: c_int) -> *const c_char;
        pub fn wrs_attn_reserve(ctx: *mut WrsCtx, r: *const WrsReserve) -> c_int;

        // host-slice drop-ins: attention.rs:68-78, :29-41, :246-254, decoder.rs:835-892
        pub fn wrs_flash_attention_2(ctx: *mut WrsCtx, q: *const f32, q_len: usize,
            k: *const f32, k_len: usize, v: *const f32, v_len: usize, t_q: usize, t_kv: usize,
            n_heads: usize, d_model: usize, causal: c_int, output: *mut f32,
            output_len: usize) -> c_int;
        pub fn wrs_multi_head_attention(ctx: *mut WrsCtx, q: *const f32, q_len: usize,
            k: *const f32, k_len: usize, v: *const f32, v_len: usize, t_q: usize, t_kv: usize,
            n_heads: usize, d_model: usize, causal: c_int, output: *mut f32,
            output_len: usize) -> c_int;
        pub fn wrs_single_token_mha_d64(ctx: *mut WrsCtx, q: *const f32, q_len: usize,
            k: *const f32, k_len: usize, v: *const f32, v_len: usize, t_kv: usize,
            n_heads: usize, d_model: usize, output: *mut f32, output_len: usize) -> c_int;
        pub fn wrs_mha_with_cache(ctx: *mut WrsCtx, q: *const f32, q_len: usize, k: *const f32,
            k_len: usize, v: *const f32, v_len: usize, n_tokens: usize, total_tokens: usize,
            t_past: usize, n_heads: usize, d_model: usize, output: *mut f32,
            output_len: usize) -> c_int;

        // device-resident prefill: encoder.rs:289-299 for every window of a batch
        pub fn wrs_attn_prefill(ctx: *mut WrsCtx, q_dtype: c_int, q: *const c_void,
            q_layout: *const WrsLayout, kv_dtype: c_int, k: *const c_void,
            k_layout: *const WrsLayout, v: *const c_void, v_layout: *const WrsLayout,
            out: *mut f32, out_layout: *const WrsLayout, batch: usize, n_heads: usize,
            t_q: usize, t_kv: usize, d_head: usize, causal: c_int,
            q_pos_offset: usize) -> c_int;

        // device KV arena: DecoderKvCache, decoder.rs:131-264
        pub fn wrs_kv_create(ctx: *mut WrsCtx, n_layers: usize, n_slots: usize, n_heads: usize,
            max_ctx: usize, n_audio_max: usize, out: *mut *mut WrsKv) -> c_int;
        // the same with the plane element type (WRS_F16 or WRS_F32)
        pub fn wrs_kv_create_dtype(ctx: *mut WrsCtx, n_layers: usize, n_slots: usize,
            n_heads: usize, max_ctx: usize, n_audio_max: usize, dtype: c_int,
            out: *mut *mut WrsKv) -> c_int;
        pub fn wrs_kv_dtype(kv: *mut WrsKv, dtype: *mut c_int) -> c_int;
        pub fn wrs_kv_destroy(kv: *mut WrsKv);
        pub fn wrs_kv_clear(kv: *mut WrsKv) -> c_int;
        pub fn wrs_kv_clear_slot(kv: *mut WrsKv, slot: usize) -> c_int;
        pub fn wrs_kv_invalidate_cross(kv: *mut WrsKv) -> c_int;
        pub fn wrs_kv_ensure_slots(kv: *mut WrsKv, n_slots: usize) -> c_int;
        pub fn wrs_kv_copy_slot(kv: *mut WrsKv, dst: usize, src: usize) -> c_int;
        pub fn wrs_kv_slot_len(kv: *mut WrsKv, slot: usize, len: *mut usize) -> c_int;
        pub fn wrs_kv_set_len(kv: *mut WrsKv, slot: usize, len: usize) -> c_int;
        pub fn wrs_kv_slide_to_fit(kv: *mut WrsKv, slot: usize, n_new: usize, max_ctx: usize,
            pos: *mut usize) -> c_int;
        pub fn wrs_kv_append(kv: *mut WrsKv, layer: usize, slot: usize, k_rows: *const f32,
            v_rows: *const f32, n: usize, src_on_host: c_int) -> c_int;
        pub fn wrs_kv_advance(kv: *mut WrsKv, slot: usize, n: usize) -> c_int;
        pub fn wrs_kv_set_cross(kv: *mut WrsKv, layer: usize, k: *const f32, v: *const f32,
            n_audio: usize, src_on_host: c_int) -> c_int;
        pub fn wrs_kv_cross_len(kv: *mut WrsKv, layer: usize, n_audio: *mut usize) -> c_int;
        pub fn wrs_kv_self_planes(kv: *mut WrsKv, k: *mut *mut c_void, v: *mut *mut c_void,
            slot_stride_elems: *mut usize) -> c_int;
        pub fn wrs_kv_cross_planes(kv: *mut WrsKv, k: *mut *mut c_void,
            v: *mut *mut c_void) -> c_int;

        // decode over the arena: decoder.rs:613-647 (self) and :689-724 (cross)
        pub fn wrs_attn_decode_self(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            slots: *const usize, n: usize, q: *const f32, out: *mut f32) -> c_int;
        pub fn wrs_attn_decode_cross(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            q: *const f32, n_beams: usize, out: *mut f32) -> c_int;
        // allocation-free decode_cross (no reference counterpart): fixed scratch,
        // for callers that cannot allocate (graph capture, serving loops)
        pub fn wrs_attn_decode_cross_noalloc(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            q: *const f32, n_beams: usize, out: *mut f32) -> c_int;
        pub fn wrs_attn_prefill_self(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            slot: usize, q: *const f32, n_tokens: usize, out: *mut f32) -> c_int;
        pub fn wrs_attn_prefill_cross(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            q: *const f32, n_tokens: usize, out: *mut f32) -> c_int;
        // the same, also writing the rows' softmax statistics for the one-pass capture
        pub fn wrs_attn_prefill_cross_lse(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            q: *const f32, n_tokens: usize, out: *mut f32, lse: *mut f32) -> c_int;

        // decoder.rs:796-828 capture_cross_attention_heads; `selected` as two arrays
        pub fn wrs_attn_capture_cross_heads(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            q: *const f32, n_tokens: usize, slots: *const usize, heads: *const usize,
            n_pairs: usize, n_selected: usize, row_offset: usize, out: *mut f32,
            out_len: usize) -> c_int;
        // one launch, with the statistics wrs_attn_prefill_cross_lse wrote for the same rows
        pub fn wrs_attn_capture_cross_heads_lse(ctx: *mut WrsCtx, kv: *mut WrsKv, layer: usize,
            q: *const f32, n_tokens: usize, slots: *const usize, heads: *const usize,
            n_pairs: usize, n_selected: usize, row_offset: usize, out: *mut f32,
            out_len: usize, lse: *const f32) -> c_int;

        // weight.rs:116-137 / quant.rs:415-473: LinearWeight::linear with f16 weights
        pub fn wrs_linear(ctx: *mut WrsCtx, x_dtype: c_int, x: *const c_void, x_len: usize,
            x_row_stride: i64, w: *const c_void, bias: *const f32, n_tokens: usize,
            n_in: usize, n_out: usize, out_dtype: c_int, out: *mut c_void, out_len: usize,
            out_row_stride: i64, out_head_stride: i64) -> c_int;
        // decoder.rs:597-611: the q, k, v linears of one normalized input, one launch
        pub fn wrs_linear_group(ctx: *mut WrsCtx, x_dtype: c_int, x: *const c_void,
            x_len: usize, x_row_stride: i64, n_groups: usize, w: *const *const c_void,
            bias: *const *const f32, n_tokens: usize, n_in: usize, n_out: usize,
            out_dtype: c_int, out: *const *mut c_void, out_len: *const usize,
            out_row_stride: i64, out_head_stride: i64) -> c_int;
        // decoder.rs:586-611 / :660-668 / :737-753: layer_norm -> linears -> gelu
        pub fn wrs_linear_fused(ctx: *mut WrsCtx, x: *const f32, x_len: usize,
            x_row_stride: i64, ln_gamma: *const f32, ln_beta: *const f32, ln_eps: f32,
            n_groups: usize, w: *const *const c_void, bias: *const *const f32,
            n_tokens: usize, n_in: usize, n_out: usize, activation: c_int, out_dtype: c_int,
            out: *const *mut c_void, out_len: *const usize, out_row_stride: i64,
            out_head_stride: i64) -> c_int;
        // norm.rs:116-143 and gelu.rs:11-23 over device f32 rows
        pub fn wrs_layer_norm(ctx: *mut WrsCtx, x: *const f32, x_len: usize,
            gamma: *const f32, beta: *const f32, eps: f32, n_tokens: usize, d_model: usize,
            out_dtype: c_int, out: *mut c_void, out_len: usize) -> c_int;
        pub fn wrs_gelu_inplace(ctx: *mut WrsCtx, data: *mut f32, n: usize) -> c_int;
        // decoder.rs:423-447 precompute_cross_attn, every layer into the arena
        pub fn wrs_kv_set_cross_proj(kv: *mut WrsKv, x_dtype: c_int, enc: *const c_void,
            enc_len: usize, enc_row_stride: i64, n_audio: usize, w_k: *const *const c_void,
            w_v: *const *const c_void, b_v: *const *const f32) -> c_int;

        // measurement helper (no reference counterpart)
        pub fn wrs_stream_read(ctx: *mut WrsCtx, src: *const c_void, bytes: usize,
            sink: *mut f32, sink_len: usize) -> c_int;
        pub fn wrs_stream_read_shape(ctx: *mut WrsCtx, src: *const c_void, bytes: usize,
            threads: c_int, loads_per_lane: c_int, sink: *mut f32, sink_len: usize) -> c_int;
    }
}

use ffi::*;

/// One context: a device, a HIP stream and scratch. Not `Sync`: a context is
/// used by one thread at a time.
pub struct AttnCtx(*mut WrsCtx);

unsafe impl Send for AttnCtx {}

impl AttnCtx {
    /// `wrs_attn_create`; panics when no such device exists.
    pub fn new(device: i32) -> Self {
        let mut p = std::ptr::null_mut();
        let rc = unsafe { wrs_attn_create(device, &mut p) };
        if rc != WRS_OK {
            panic!("wrs_attn_create(device {device}) failed: {}", status_text(rc));
        }
        AttnCtx(p)
    }

    pub fn raw(&self) -> *mut WrsCtx {
        self.0
    }

    /// Status code -> the reference's contract: success returns, a shape
    /// violation panics with the message the reference's `assert!` would give
    /// (`WRS_EINVAL`), any other failure panics with the library's text.
    pub fn check(&self, rc: c_int) {
        if rc != WRS_OK {
            let msg = unsafe { CStr::from_ptr(wrs_attn_last_error(self.0)) }.to_string_lossy();
            if rc == WRS_EINVAL {
                panic!("{msg}");
            }
            panic!("{}: {msg}", status_text(rc));
        }
    }

    pub fn reserve(&self, r: &WrsReserve) {
        self.check(unsafe { wrs_attn_reserve(self.0, r) });
    }

    pub fn synchronize(&self) {
        self.check(unsafe { wrs_attn_synchronize(self.0) });
    }

    /// attention.rs:68-78 on host slices (synchronous).
    pub fn flash_attention_2(&self, q: &[f32], k: &[f32], v: &[f32], t_q: usize, t_kv: usize,
                             n_heads: usize, d_model: usize, causal: bool, output: &mut [f32]) {
        self.check(unsafe {
            wrs_flash_attention_2(self.0, q.as_ptr(), q.len(), k.as_ptr(), k.len(), v.as_ptr(),
                                  v.len(), t_q, t_kv, n_heads, d_model, causal as c_int,
                                  output.as_mut_ptr(), output.len())
        });
    }

    /// attention.rs:29-41 on host slices (synchronous).
    pub fn multi_head_attention(&self, q: &[f32], k: &[f32], v: &[f32], t_q: usize,
                                t_kv: usize, n_heads: usize, d_model: usize, causal: bool,
                                output: &mut [f32]) {
        self.check(unsafe {
            wrs_multi_head_attention(self.0, q.as_ptr(), q.len(), k.as_ptr(), k.len(),
                                     v.as_ptr(), v.len(), t_q, t_kv, n_heads, d_model,
                                     causal as c_int, output.as_mut_ptr(), output.len())
        });
    }

    /// attention.rs:246-254 on host slices (synchronous).
    pub fn single_token_mha_d64(&self, q: &[f32], k: &[f32], v: &[f32], t_kv: usize,
                                n_heads: usize, d_model: usize, output: &mut [f32]) {
        self.check(unsafe {
            wrs_single_token_mha_d64(self.0, q.as_ptr(), q.len(), k.as_ptr(), k.len(),
                                     v.as_ptr(), v.len(), t_kv, n_heads, d_model,
                                     output.as_mut_ptr(), output.len())
        });
    }

    /// decoder.rs:835-892 on host slices (synchronous).
    pub fn multi_head_attention_with_cache(&self, q: &[f32], k: &[f32], v: &[f32],
                                           n_tokens: usize, total_tokens: usize, t_past: usize,
                                           n_heads: usize, d_model: usize, output: &mut [f32]) {
        self.check(unsafe {
            wrs_mha_with_cache(self.0, q.as_ptr(), q.len(), k.as_ptr(), k.len(), v.as_ptr(),
                               v.len(), n_tokens, total_tokens, t_past, n_heads, d_model,
                               output.as_mut_ptr(), output.len())
        });
    }
}

impl Drop for AttnCtx {
    fn drop(&mut self) {
        unsafe { wrs_attn_destroy(self.0) }
    }
}

/// The device KV arena of one context (`DecoderKvCache` in HBM). Device
/// pointers passed to its methods must come from the same device.
pub struct KvArena<'c> {
    ctx: &'c AttnCtx,
    kv: *mut WrsKv,
}

impl<'c> KvArena<'c> {
    /// DecoderKvCache::new (decoder.rs:148-157) with a fixed capacity.
    pub fn new(ctx: &'c AttnCtx, n_layers: usize, n_slots: usize, n_heads: usize,
               max_ctx: usize, n_audio_max: usize) -> Self {
        let mut kv = std::ptr::null_mut();
        ctx.check(unsafe {
            wrs_kv_create(ctx.raw(), n_layers, n_slots, n_heads, max_ctx, n_audio_max, &mut kv)
        });
        KvArena { ctx, kv }
    }

    /// The same with f32 planes (`ffi::WRS_F32`): the reference cache's own
    /// values, attention with the reference's arithmetic.
    pub fn new_with_dtype(ctx: &'c AttnCtx, n_layers: usize, n_slots: usize, n_heads: usize,
                          max_ctx: usize, n_audio_max: usize, dtype: c_int) -> Self {
        let mut kv = std::ptr::null_mut();
        ctx.check(unsafe {
            wrs_kv_create_dtype(ctx.raw(), n_layers, n_slots, n_heads, max_ctx, n_audio_max,
                                dtype, &mut kv)
        });
        KvArena { ctx, kv }
    }

    pub fn raw(&self) -> *mut WrsKv {
        self.kv
    }

    pub fn clear(&self) {
        self.ctx.check(unsafe { wrs_kv_clear(self.kv) });
    }
    pub fn clear_slot(&self, slot: usize) {
        self.ctx.check(unsafe { wrs_kv_clear_slot(self.kv, slot) });
    }
    pub fn invalidate_cross(&self) {
        self.ctx.check(unsafe { wrs_kv_invalidate_cross(self.kv) });
    }
    pub fn ensure_slots(&self, n_slots: usize) {
        self.ctx.check(unsafe { wrs_kv_ensure_slots(self.kv, n_slots) });
    }
    pub fn copy_slot(&self, dst: usize, src: usize) {
        self.ctx.check(unsafe { wrs_kv_copy_slot(self.kv, dst, src) });
    }
    pub fn slot_len(&self, slot: usize) -> usize {
        let mut n = 0usize;
        self.ctx.check(unsafe { wrs_kv_slot_len(self.kv, slot, &mut n) });
        n
    }
    pub fn set_len(&self, slot: usize, len: usize) {
        self.ctx.check(unsafe { wrs_kv_set_len(self.kv, slot, len) });
    }
    pub fn slide_to_fit(&self, slot: usize, n_new: usize, max_ctx: usize) -> usize {
        let mut pos = 0usize;
        self.ctx.check(unsafe { wrs_kv_slide_to_fit(self.kv, slot, n_new, max_ctx, &mut pos) });
        pos
    }
    pub fn advance(&self, slot: usize, n: usize) {
        self.ctx.check(unsafe { wrs_kv_advance(self.kv, slot, n) });
    }
    pub fn cross_len(&self, layer: usize) -> usize {
        let mut n = 0usize;
        self.ctx.check(unsafe { wrs_kv_cross_len(self.kv, layer, &mut n) });
        n
    }
    /// decoder.rs:631-635 from host rows `[n][d_model]` (synchronous).
    pub fn append_host(&self, layer: usize, slot: usize, k_rows: &[f32], v_rows: &[f32],
                       n: usize) {
        self.ctx.check(unsafe {
            wrs_kv_append(self.kv, layer, slot, k_rows.as_ptr(), v_rows.as_ptr(), n, 1)
        });
    }
    /// decoder.rs:423-447's stored K/V of one layer, from host rows (synchronous).
    pub fn set_cross_host(&self, layer: usize, k: &[f32], v: &[f32], n_audio: usize) {
        self.ctx.check(unsafe {
            wrs_kv_set_cross(self.kv, layer, k.as_ptr(), v.as_ptr(), n_audio, 1)
        });
    }
    /// One self-attention decode launch for every row (asynchronous).
    ///
    /// # Safety
    /// `q` and `out` are device pointers of `slots.len() * d_model` f32.
    pub unsafe fn decode_self(&self, layer: usize, slots: &[usize], q: *const f32,
                              out: *mut f32) {
        self.ctx.check(wrs_attn_decode_self(self.ctx.raw(), self.kv, layer, slots.as_ptr(),
                                            slots.len(), q, out));
    }
    /// One cross-attention decode launch for all beams (asynchronous).
    ///
    /// # Safety
    /// `q` and `out` are device pointers of `n_beams * d_model` f32.
    pub unsafe fn decode_cross(&self, layer: usize, q: *const f32, n_beams: usize,
                               out: *mut f32) {
        self.ctx.check(wrs_attn_decode_cross(self.ctx.raw(), self.kv, layer, q, n_beams, out));
    }
    /// `decode_cross` on the library's fixed device scratch: allocates nothing
    /// (usable under graph capture); calls on one GPU must not overlap.
    ///
    /// # Safety
    /// As for [`KvArena::decode_cross`].
    pub unsafe fn decode_cross_noalloc(&self, layer: usize, q: *const f32, n_beams: usize,
                                       out: *mut f32) {
        self.ctx.check(wrs_attn_decode_cross_noalloc(self.ctx.raw(), self.kv, layer, q,
                                                     n_beams, out));
    }
    /// decoder.rs:698-708's cross-attention of `n_tokens` prompt rows, also
    /// writing the rows' softmax statistics for [`KvArena::capture_cross_heads_lse`].
    ///
    /// # Safety
    /// `q` and `out` are device pointers of `n_tokens * d_model` f32, `lse` of
    /// `2 * n_heads * n_tokens` f32.
    pub unsafe fn prefill_cross_lse(&self, layer: usize, q: *const f32, n_tokens: usize,
                                    out: *mut f32, lse: *mut f32) {
        self.ctx.check(wrs_attn_prefill_cross_lse(self.ctx.raw(), self.kv, layer, q, n_tokens,
                                                  out, lse));
    }
    /// decoder.rs:709-721's alignment-head capture in one launch, from the
    /// statistics `prefill_cross_lse` wrote for the same rows; `selected` holds
    /// (slot, head) pairs as the reference's `layer_heads` does.
    ///
    /// # Safety
    /// `q` is a device pointer of `n_tokens * d_model` f32, `out` of `out_len` f32,
    /// `lse` as written by `prefill_cross_lse` for these rows.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn capture_cross_heads_lse(&self, layer: usize, q: *const f32, n_tokens: usize,
                                          selected: &[(usize, usize)], n_selected: usize,
                                          row_offset: usize, out: *mut f32, out_len: usize,
                                          lse: *const f32) {
        let slots: Vec<usize> = selected.iter().map(|&(s, _)| s).collect();
        let heads: Vec<usize> = selected.iter().map(|&(_, h)| h).collect();
        self.ctx.check(wrs_attn_capture_cross_heads_lse(self.ctx.raw(), self.kv, layer, q,
                                                        n_tokens, slots.as_ptr(),
                                                        heads.as_ptr(), selected.len(),
                                                        n_selected, row_offset, out, out_len,
                                                        lse));
    }
}

impl Drop for KvArena<'_> {
    fn drop(&mut self) {
        unsafe { wrs_kv_destroy(self.kv) }
    }
}

fn status_text(rc: c_int) -> String {
    unsafe { CStr::from_ptr(wrs_attn_status_string(rc)) }.to_string_lossy().into_owned()
}

// ---------------------------------------------------------------------------
// Process-wide device selection, per-thread contexts, and the reference
// signatures the `cfg(feature = "hip")` branches of whisper-tensor forward to.
// ---------------------------------------------------------------------------

static DEVICE: AtomicI32 = AtomicI32::new(-1);

thread_local! {
    /// This thread's context and the device it was created on.
    static CTX: RefCell<Option<(i32, AttnCtx)>> = const { RefCell::new(None) };
}

/// Route the attention entry points to GPU `device` (`Some`) or back to the
/// CPU path (`None`). Threads create their context on first use.
pub fn set_device(device: Option<i32>) {
    DEVICE.store(device.map_or(-1, |d| d.max(0)), Ordering::SeqCst);
}

/// True when a device is selected: the `cfg(feature = "hip")` branches test
/// this and otherwise fall through to the reference's CPU body.
pub fn enabled() -> bool {
    DEVICE.load(Ordering::Relaxed) >= 0
}

/// Runs `f` on this thread's context for the selected device (created on the
/// thread's first call, replaced when the selection changes).
pub fn with_ctx<R>(f: impl FnOnce(&AttnCtx) -> R) -> R {
    let dev = DEVICE.load(Ordering::Relaxed);
    assert!(dev >= 0, "whisper-tensor-hip: no GPU selected (set_device)");
    CTX.with(|cell| {
        let mut slot = cell.borrow_mut();
        if !matches!(slot.as_ref(), Some((d, _)) if *d == dev) {
            *slot = Some((dev, AttnCtx::new(dev)));
        }
        f(&slot.as_ref().unwrap().1)
    })
}

/// `whisper_tensor::ops::flash_attention_2` (attention.rs:68-78).
pub fn flash_attention_2(q: &[f32], k: &[f32], v: &[f32], t_q: usize, t_kv: usize,
                         n_heads: usize, d_model: usize, causal: bool, output: &mut [f32]) {
    with_ctx(|c| c.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, causal, output))
}

/// `whisper_tensor::ops::multi_head_attention` (attention.rs:29-41).
pub fn multi_head_attention(q: &[f32], k: &[f32], v: &[f32], t_q: usize, t_kv: usize,
                            n_heads: usize, d_model: usize, causal: bool, output: &mut [f32]) {
    with_ctx(|c| c.multi_head_attention(q, k, v, t_q, t_kv, n_heads, d_model, causal, output))
}

/// `whisper_tensor::ops::single_token_mha_d64` (attention.rs:246-254).
pub fn single_token_mha_d64(q: &[f32], k: &[f32], v: &[f32], t_kv: usize, n_heads: usize,
                            d_model: usize, output: &mut [f32]) {
    with_ctx(|c| c.single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, output))
}

/// The decoder's `multi_head_attention_with_cache` (decoder.rs:835-845).
pub fn multi_head_attention_with_cache(q: &[f32], k: &[f32], v: &[f32], n_tokens: usize,
                                       total_tokens: usize, t_past: usize, n_heads: usize,
                                       d_model: usize, output: &mut [f32]) {
    with_ctx(|c| {
        c.multi_head_attention_with_cache(q, k, v, n_tokens, total_tokens, t_past, n_heads,
                                          d_model, output)
    })
}

/// Dispatch rule of the device-resident prefill for callers holding device
/// tensors: `c_void` pointers with a `WrsLayout` each (see the header).
///
/// # Safety
/// All pointers are device pointers valid for the described views.
pub unsafe fn prefill(ctx: &AttnCtx, q_dtype: c_int, q: *const c_void, q_layout: &WrsLayout,
                      kv_dtype: c_int, k: *const c_void, k_layout: &WrsLayout,
                      v: *const c_void, v_layout: &WrsLayout, out: *mut f32,
                      out_layout: &WrsLayout, batch: usize, n_heads: usize, t_q: usize,
                      t_kv: usize, d_head: usize, causal: bool, q_pos_offset: usize) {
    ctx.check(wrs_attn_prefill(ctx.raw(), q_dtype, q, q_layout, kv_dtype, k, k_layout, v,
                               v_layout, out, out_layout, batch, n_heads, t_q, t_kv, d_head,
                               causal as c_int, q_pos_offset));
}
