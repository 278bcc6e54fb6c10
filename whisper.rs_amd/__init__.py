"""whisper.rs attention path on AMD Instinct MI355X (gfx950).

Host-side mirror of the reference's attention interface over the C ABI of
``include/wrs_attn.h`` (library ``lib/libwrs_attn.so``):

* reference-named host-slice functions with the reference's argument meaning
  and error behaviour -- ``flash_attention_2`` / ``multi_head_attention``
  (crates/tensor/src/ops/attention.rs:29-243), ``single_token_mha_d64``
  (attention.rs:246-434) and ``mha_with_cache``
  (crates/whisper/src/decoder.rs:835-892). They take float32 numpy arrays;
  a shape violation that panics in the reference raises ``AssertionError``.
* device-resident entry points on torch tensors (torch supplies device memory
  and the stream; every FLOP runs in this package's HIP kernels):
  ``prefill`` and the ``KvArena`` (DecoderKvCache, decoder.rs:131-264) with
  its ``decode_self`` / ``decode_cross`` / ``prefill_self`` / ``prefill_cross``
  and the DTW alignment-head capture ``capture_cross_heads``.

There is no CPU fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _lib as _L
from ._lib import (WRS_BF16, WRS_EINVAL, WRS_F16, WRS_F32, WRS_OK, ExtensionMissing, Layout,
                   header_symbols)

Q_TILE = 128  # crates/tensor/src/ops/attention.rs:13 (reference tile constants)
KV_TILE = 128  # crates/tensor/src/ops/attention.rs:26

__all__ = [
    "Context", "KvArena", "ExtensionMissing", "Layout", "flash_attention_2",
    "multi_head_attention", "single_token_mha_d64", "mha_with_cache", "prefill",
    "token_major", "default_context", "header_symbols", "Q_TILE", "KV_TILE", "linear",
    "linear_group", "linear_fused", "layer_norm", "gelu_inplace",
]


class Context:
    """One device, one stream, private scratch (``wrs_attn_ctx``)."""

    def __init__(self, device: int = 0):
        self._lib = _L.lib()
        h = ctypes.c_void_p()
        rc = self._lib.wrs_attn_create(int(device), ctypes.byref(h))
        if rc != WRS_OK:
            raise RuntimeError(f"wrs_attn_create(device={device}) failed: "
                               f"{_L.status_string(rc)}")
        self.handle = h
        self.device = int(device)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.wrs_attn_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc: int, what: str) -> None:
        if rc == WRS_OK:
            return
        msg = self._lib.wrs_attn_last_error(self.handle).decode()
        if rc == WRS_EINVAL:
            # The reference panics on these (assert!/assert_eq!).
            raise AssertionError(f"{what}: {msg}")
        raise RuntimeError(f"{what}: {_L.status_string(rc)}: {msg}")

    def set_stream(self, stream_handle: int | None) -> None:
        """Queue work on a hipStream_t handle; 0/None is the null stream."""
        self.check(self._lib.wrs_attn_set_stream(self.handle, stream_handle or None),
                   "wrs_attn_set_stream")

    def use_torch_stream(self) -> None:
        """Queue work on torch's current stream of this device."""
        import torch
        self.set_stream(torch.cuda.current_stream(self.device).cuda_stream)

    def set_schedule(self, prefill_queries: int = 0, f32_split: int = -1) -> None:
        """Work decomposition of this context's prefill calls
        (``wrs_attn_set_schedule``): queries per workgroup of the f16/bf16
        kernel (256 or 128; -256, -192 or -128 for key halves on 8 or 12
        waves; -2 or -3 for 128-query blocks split over that many such
        workgroups; 32 for the key split; 0 = by grid size) and the f32
        kernel's key split (-1 = by grid size, 0 = 128-query blocks, 1..4 =
        key split over four or that many waves, 5 = the four-wave key split
        with each block over several workgroups)."""
        self.check(self._lib.wrs_attn_set_schedule(self.handle, int(prefill_queries),
                                                   int(f32_split)), "wrs_attn_set_schedule")

    def synchronize(self) -> None:
        self.check(self._lib.wrs_attn_synchronize(self.handle), "wrs_attn_synchronize")

    def reserve(self, **sizes) -> None:
        """Size the context scratch for the largest calls it will serve
        (``wrs_attn_reserve``): n_heads, decode_rows, decode_keys,
        capture_tokens, capture_keys, linear_tokens, linear_n_in."""
        r = _L.Reserve(**{k: int(v) for k, v in sizes.items()})
        self.check(self._lib.wrs_attn_reserve(self.handle, ctypes.byref(r)), "wrs_attn_reserve")


_default = None
_default_lock = threading.Lock()


def default_context() -> Context:
    global _default
    with _default_lock:
        if _default is None:
            _default = Context(0)
        return _default


# --------------------------------------------------------------------------
# host-slice drop-ins (reference signatures)
# --------------------------------------------------------------------------

def _f32(a, name):
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]):
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    return a.ctypes.data_as(ctypes.c_void_p), a.size


def flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, causal, output, ctx=None):
    """crates/tensor/src/ops/attention.rs:68-78 on the GPU (synchronous)."""
    ctx = ctx or default_context()
    (pq, nq), (pk, nk), (pv, nv), (po, no) = (_f32(q, "q"), _f32(k, "k"), _f32(v, "v"),
                                              _f32(output, "output"))
    ctx.check(ctx._lib.wrs_flash_attention_2(ctx.handle, pq, nq, pk, nk, pv, nv, t_q, t_kv,
                                             n_heads, d_model, int(bool(causal)), po, no),
              "flash_attention_2")


def multi_head_attention(q, k, v, t_q, t_kv, n_heads, d_model, causal, output, ctx=None):
    """crates/tensor/src/ops/attention.rs:29-41 on the GPU (synchronous)."""
    ctx = ctx or default_context()
    (pq, nq), (pk, nk), (pv, nv), (po, no) = (_f32(q, "q"), _f32(k, "k"), _f32(v, "v"),
                                              _f32(output, "output"))
    ctx.check(ctx._lib.wrs_multi_head_attention(ctx.handle, pq, nq, pk, nk, pv, nv, t_q, t_kv,
                                                n_heads, d_model, int(bool(causal)), po, no),
              "multi_head_attention")


def single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, output, ctx=None):
    """crates/tensor/src/ops/attention.rs:246-254 on the GPU (synchronous)."""
    ctx = ctx or default_context()
    (pq, nq), (pk, nk), (pv, nv), (po, no) = (_f32(q, "q"), _f32(k, "k"), _f32(v, "v"),
                                              _f32(output, "output"))
    ctx.check(ctx._lib.wrs_single_token_mha_d64(ctx.handle, pq, nq, pk, nk, pv, nv, t_kv,
                                                n_heads, d_model, po, no),
              "single_token_mha_d64")


def mha_with_cache(q, k, v, n_tokens, total_tokens, t_past, n_heads, d_model, output, ctx=None):
    """crates/whisper/src/decoder.rs:835-892 on the GPU (synchronous)."""
    ctx = ctx or default_context()
    (pq, nq), (pk, nk), (pv, nv), (po, no) = (_f32(q, "q"), _f32(k, "k"), _f32(v, "v"),
                                              _f32(output, "output"))
    ctx.check(ctx._lib.wrs_mha_with_cache(ctx.handle, pq, nq, pk, nk, pv, nv, n_tokens,
                                          total_tokens, t_past, n_heads, d_model, po, no),
              "multi_head_attention_with_cache")


# --------------------------------------------------------------------------
# device-resident entry points (torch tensors as device memory)
# --------------------------------------------------------------------------

_DT = {"torch.float32": WRS_F32, "torch.float16": WRS_F16, "torch.bfloat16": WRS_BF16}


def _dtype_code(t):
    try:
        return _DT[str(t.dtype)]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def token_major(t_rows: int, d_model: int, d_head: int, row_stride: int | None = None) -> Layout:
    """Layout of the reference's [T][d_model] rows (optionally inside wider rows)."""
    rs = d_model if row_stride is None else row_stride
    return Layout(t_rows * rs, d_head, rs)


def prefill(q, k, v, out, *, batch, n_heads, t_q, t_kv, d_head, q_layout, kv_layout, out_layout,
            causal=False, q_pos_offset=0, k_layout=None, ctx=None):
    """Batched flash_attention_2 over device tensors (asynchronous on ctx's stream)."""
    ctx = ctx or default_context()
    if out.dtype.__str__() != "torch.float32":
        raise TypeError("out must be float32")
    kl = k_layout or kv_layout
    ctx.check(ctx._lib.wrs_attn_prefill(
        ctx.handle, _dtype_code(q), q.data_ptr(), ctypes.byref(q_layout), _dtype_code(k),
        k.data_ptr(), ctypes.byref(kl), v.data_ptr(), ctypes.byref(kv_layout), out.data_ptr(),
        ctypes.byref(out_layout), batch, n_heads, t_q, t_kv, d_head, int(bool(causal)),
        q_pos_offset), "wrs_attn_prefill")


def linear(x, w, bias, out, *, out_row_stride=None, out_head_stride=64, ctx=None):
    """LinearWeight::linear with f16 weights (crates/tensor/src/weight.rs:116-137,
    crates/tensor/src/ops/quant.rs:415-473): out(t, r) = w[r] . x[t] + bias[r].

    ``x`` [n_tokens][n_in] float32 or float16, ``w`` [n_out][n_in] float16,
    ``bias`` float32 [n_out] or None, all CUDA tensors. ``out`` (float32,
    float16 or bfloat16) receives out(t, r) at
    t*out_row_stride + (r // 64)*out_head_stride + r % 64 elements from its start;
    the defaults give token-major [n_tokens][n_out] rows.
    """
    ctx = ctx or default_context()
    n_tokens, n_in = x.shape[0], x.shape[-1]
    n_out = w.shape[0]
    assert w.shape[1] == n_in and str(w.dtype) == "torch.float16"  # quant.rs:440
    if bias is not None:
        assert bias.numel() == n_out and str(bias.dtype) == "torch.float32"  # quant.rs:427
    rs = n_out if out_row_stride is None else out_row_stride
    ctx.check(_L.lib().wrs_linear(ctx.handle, _dtype_code(x), x.data_ptr(), _span(x),
                                  x.stride(0) if x.dim() > 1 else n_in, w.data_ptr(),
                                  None if bias is None else bias.data_ptr(), n_tokens, n_in,
                                  n_out, _dtype_code(out), out.data_ptr(), _span(out), rs,
                                  out_head_stride), "linear")


def linear_group(x, ws, biases, outs, *, out_row_stride=None, out_head_stride=64, ctx=None):
    """Several LinearWeight::linear projections of one input in one launch
    (the self-attention q, k, v of crates/whisper/src/decoder.rs:597-611):
    ``outs[g]`` = ``x`` W_g^T + ``biases[g]``, each exactly as :func:`linear`.
    ``ws`` are float16 [n_out][n_in] CUDA tensors of one shape; ``biases`` is
    None or a list with float32 tensors or None entries; ``outs`` share dtype
    and shape."""
    ctx = ctx or default_context()
    n = len(ws)
    assert n == len(outs) and n > 0
    n_tokens, n_in = x.shape[0], x.shape[-1]
    n_out = ws[0].shape[0]
    for w in ws:
        assert tuple(w.shape) == (n_out, n_in) and str(w.dtype) == "torch.float16"
    biases = list(biases) if biases is not None else [None] * n
    for b in biases:
        assert b is None or (b.numel() == n_out and str(b.dtype) == "torch.float32")
    for o in outs:
        assert o.dtype == outs[0].dtype
    rs = n_out if out_row_stride is None else out_row_stride
    vp = ctypes.c_void_p
    w_arr = (vp * n)(*[w.data_ptr() for w in ws])
    b_arr = (vp * n)(*[None if b is None else b.data_ptr() for b in biases])
    o_arr = (vp * n)(*[o.data_ptr() for o in outs])
    len_arr = (ctypes.c_size_t * n)(*[_span(o) for o in outs])
    ctx.check(_L.lib().wrs_linear_group(ctx.handle, _dtype_code(x), x.data_ptr(), _span(x),
                                        x.stride(0) if x.dim() > 1 else n_in, n, w_arr, b_arr,
                                        n_tokens, n_in, n_out, _dtype_code(outs[0]), o_arr,
                                        len_arr, rs, out_head_stride), "linear_group")


def linear_fused(x, ws, biases, outs, *, ln=None, act=None, out_row_stride=None,
                 out_head_stride=64, ctx=None):
    """layer_norm -> linear (one or more weight groups) -> GELU in one launch for
    decode-sized batches (decoder.rs:586-611, :660-668, :737-753).

    ``x`` float32 [n_tokens][n_in]; ``ln`` None or (gamma, beta, eps) with float32
    CUDA tensors of n_in values; ``act`` None or "gelu". The values equal
    :func:`layer_norm` (float32 out), then :func:`linear_group`, then
    :func:`gelu_inplace` on each output, the GELU taken in float32 before any
    rounding to ``outs``' dtype."""
    ctx = ctx or default_context()
    assert str(x.dtype) == "torch.float32"
    n = len(ws)
    assert n == len(outs) and n > 0
    n_tokens, n_in = x.shape[0], x.shape[-1]
    n_out = ws[0].shape[0]
    for w in ws:
        assert tuple(w.shape) == (n_out, n_in) and str(w.dtype) == "torch.float16"
    biases = list(biases) if biases is not None else [None] * n
    for b in biases:
        assert b is None or (b.numel() == n_out and str(b.dtype) == "torch.float32")
    for o in outs:
        assert o.dtype == outs[0].dtype
    if ln is not None:
        gamma, beta, eps = ln
        assert gamma.numel() == n_in and beta.numel() == n_in  # norm.rs:123-124
    else:
        gamma, beta, eps = None, None, 0.0
    codes = {None: 0, "gelu": 1}
    rs = n_out if out_row_stride is None else out_row_stride
    vp = ctypes.c_void_p
    w_arr = (vp * n)(*[w.data_ptr() for w in ws])
    b_arr = (vp * n)(*[None if b is None else b.data_ptr() for b in biases])
    o_arr = (vp * n)(*[o.data_ptr() for o in outs])
    len_arr = (ctypes.c_size_t * n)(*[_span(o) for o in outs])
    ctx.check(_L.lib().wrs_linear_fused(
        ctx.handle, x.data_ptr(), _span(x), x.stride(0) if x.dim() > 1 else n_in,
        None if gamma is None else gamma.data_ptr(), None if beta is None else beta.data_ptr(),
        float(eps), n, w_arr, b_arr, n_tokens, n_in, n_out, codes[act], _dtype_code(outs[0]),
        o_arr, len_arr, rs, out_head_stride), "linear_fused")


def layer_norm(x, gamma, beta, eps, out, ctx=None):
    """layer_norm (crates/tensor/src/ops/norm.rs:116-143) over the rows of the
    float32 CUDA tensor x ([num_tokens][d_model]); out float32/float16/bfloat16."""
    ctx = ctx or default_context()
    d = x.shape[-1]
    n = x.numel() // d if d else 0
    ctx.check(_L.lib().wrs_layer_norm(ctx.handle, x.data_ptr(), x.numel(), gamma.data_ptr(),
                                      beta.data_ptr(), eps, n, d, _dtype_code(out),
                                      out.data_ptr(), out.numel()), "layer_norm")


def gelu_inplace(data, ctx=None):
    """gelu_inplace (crates/tensor/src/ops/gelu.rs:11-23) on a float32 CUDA tensor."""
    ctx = ctx or default_context()
    assert str(data.dtype) == "torch.float32" and data.is_contiguous()
    ctx.check(_L.lib().wrs_gelu_inplace(ctx.handle, data.data_ptr(), data.numel()),
              "gelu_inplace")


def _span(t) -> int:
    """Elements addressable from t.data_ptr() to the end of t's storage."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


class KvArena:
    """Device KV cache (``wrs_kv``), methods named after DecoderKvCache."""

    def __init__(self, n_layers, n_slots, n_heads, max_ctx, n_audio_max, ctx=None,
                 dtype=WRS_F16):
        """dtype WRS_F16 (default) or WRS_F32: the plane element type (WRS_F32
        keeps the reference cache's f32 values and runs its arithmetic)."""
        self.ctx = ctx or default_context()
        self._lib = self.ctx._lib
        h = ctypes.c_void_p()
        self.ctx.check(self._lib.wrs_kv_create_dtype(self.ctx.handle, n_layers, n_slots,
                                                     n_heads, max_ctx, n_audio_max, dtype,
                                                     ctypes.byref(h)),
                       "wrs_kv_create")
        self.handle = h
        self.dtype = dtype
        self.n_layers, self.n_slots, self.n_heads = n_layers, n_slots, n_heads
        self.max_ctx, self.n_audio_max = max_ctx, n_audio_max
        self.d_model = n_heads * 64

    def plane_dtype(self) -> int:
        """Plane element type as the library reports it (WRS_F16 or WRS_F32)."""
        d = ctypes.c_int()
        self._c(self._lib.wrs_kv_dtype(self.handle, ctypes.byref(d)), "dtype")
        return d.value

    def close(self):
        if getattr(self, "handle", None):
            self._lib.wrs_kv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _c(self, rc, what):
        self.ctx.check(rc, what)

    # DecoderKvCache methods (decoder.rs:162-263)
    def clear(self):
        self._c(self._lib.wrs_kv_clear(self.handle), "clear")

    def clear_slot(self, slot):
        self._c(self._lib.wrs_kv_clear_slot(self.handle, slot), "clear_slot")

    def invalidate_cross(self):
        self._c(self._lib.wrs_kv_invalidate_cross(self.handle), "invalidate_cross")

    def ensure_slots(self, n_slots):
        self._c(self._lib.wrs_kv_ensure_slots(self.handle, n_slots), "ensure_slots")
        self.n_slots = max(self.n_slots, n_slots)

    def copy_slot(self, dst, src):
        self._c(self._lib.wrs_kv_copy_slot(self.handle, dst, src), "copy_slot")

    def slot_len(self, slot) -> int:
        n = ctypes.c_size_t()
        self._c(self._lib.wrs_kv_slot_len(self.handle, slot, ctypes.byref(n)), "slot_len")
        return n.value

    def set_len(self, slot, n):
        self._c(self._lib.wrs_kv_set_len(self.handle, slot, n), "set_len")

    def slide_to_fit(self, slot, n_new, max_ctx) -> int:
        pos = ctypes.c_size_t()
        self._c(self._lib.wrs_kv_slide_to_fit(self.handle, slot, n_new, max_ctx,
                                              ctypes.byref(pos)), "slide_to_fit")
        return pos.value

    @staticmethod
    def _src(t):
        if isinstance(t, np.ndarray):
            p, n = _f32(t, "rows")
            return p, n, 1
        if str(t.dtype) != "torch.float32" or not t.is_contiguous():
            raise TypeError("rows must be contiguous float32")
        return t.data_ptr(), t.numel(), 0

    def append(self, layer, slot, k_rows, v_rows):
        pk, nk, host = self._src(k_rows)
        pv, nv, host2 = self._src(v_rows)
        assert nk == nv and nk % self.d_model == 0 and host == host2
        self._c(self._lib.wrs_kv_append(self.handle, layer, slot, pk, pv, nk // self.d_model,
                                        host), "append")

    def advance(self, slot, n):
        self._c(self._lib.wrs_kv_advance(self.handle, slot, n), "advance")

    def set_cross(self, layer, k, v):
        pk, nk, host = self._src(k)
        pv, nv, host2 = self._src(v)
        assert nk == nv and nk % self.d_model == 0 and host == host2
        self._c(self._lib.wrs_kv_set_cross(self.handle, layer, pk, pv, nk // self.d_model, host),
                "set_cross")

    def cross_len(self, layer: int = 0) -> int:
        """n_audio of one layer's cross K/V (0 when not set or invalidated)."""
        n = ctypes.c_size_t()
        self._c(self._lib.wrs_kv_cross_len(self.handle, layer, ctypes.byref(n)), "cross_len")
        return n.value

    def plane_pointers(self):
        ks, vs, kc, vc = (ctypes.c_void_p() for _ in range(4))
        stride = ctypes.c_size_t()
        self._c(self._lib.wrs_kv_self_planes(self.handle, ctypes.byref(ks), ctypes.byref(vs),
                                             ctypes.byref(stride)), "self_planes")
        self._c(self._lib.wrs_kv_cross_planes(self.handle, ctypes.byref(kc), ctypes.byref(vc)),
                "cross_planes")
        return ks.value, vs.value, kc.value, vc.value

    # attention over the arena
    def decode_self(self, layer, slots, q, out):
        arr = (ctypes.c_size_t * len(slots))(*slots)
        self._c(self._lib.wrs_attn_decode_self(self.ctx.handle, self.handle, layer, arr,
                                               len(slots), q.data_ptr(), out.data_ptr()),
                "decode_self")

    def decode_cross(self, layer, q, out, n_beams=None):
        n = q.shape[0] if n_beams is None else n_beams
        self._c(self._lib.wrs_attn_decode_cross(self.ctx.handle, self.handle, layer,
                                                q.data_ptr(), n, out.data_ptr()),
                "decode_cross")

    def decode_cross_noalloc(self, layer, q, out, n_beams=None):
        """decode_cross on the library's fixed device scratch: allocates nothing."""
        n = q.shape[0] if n_beams is None else n_beams
        self._c(self._lib.wrs_attn_decode_cross_noalloc(self.ctx.handle, self.handle, layer,
                                                        q.data_ptr(), n, out.data_ptr()),
                "decode_cross_noalloc")

    def prefill_self(self, layer, slot, q, out):
        self._c(self._lib.wrs_attn_prefill_self(self.ctx.handle, self.handle, layer, slot,
                                                q.data_ptr(), q.shape[0], out.data_ptr()),
                "prefill_self")

    def prefill_cross(self, layer, q, out, lse=None):
        """Cross-attention of prompt rows (decoder.rs:698-708). With ``lse`` (a
        float32 device tensor of n_heads * n_tokens * 2 values) the rows' softmax
        statistics are written too, for ``capture_cross_heads(..., lse=lse)``."""
        if lse is None:
            self._c(self._lib.wrs_attn_prefill_cross(self.ctx.handle, self.handle, layer,
                                                     q.data_ptr(), q.shape[0], out.data_ptr()),
                    "prefill_cross")
            return
        import torch
        assert lse.dtype == torch.float32 and lse.numel() >= 2 * self.n_heads * q.shape[0]
        self._c(self._lib.wrs_attn_prefill_cross_lse(self.ctx.handle, self.handle, layer,
                                                     q.data_ptr(), q.shape[0], out.data_ptr(),
                                                     lse.data_ptr()),
                "prefill_cross_lse")

    def set_cross_proj(self, enc, w_k, w_v, b_v=None):
        """precompute_cross_attn (crates/whisper/src/decoder.rs:423-447) into the
        arena: per layer K = enc w_k^T, V = enc w_v^T + b_v, stored in the
        arena's planes (rounded to f16, or as computed for f32 arenas). ``enc`` [n_audio][d_model] float32/float16, ``w_k``/``w_v``
        lists of [d_model][d_model] float16 tensors, ``b_v`` list of float32."""
        n = len(w_k)
        assert n == len(w_v) and (b_v is None or len(b_v) == n)
        arr = ctypes.c_void_p * max(n, 1)
        wk = arr(*[t.data_ptr() for t in w_k])
        wv = arr(*[t.data_ptr() for t in w_v])
        bv = None if b_v is None else arr(*[0 if t is None else t.data_ptr() for t in b_v])
        self._c(self._lib.wrs_kv_set_cross_proj(self.handle, _dtype_code(enc), enc.data_ptr(),
                                                _span(enc), enc.stride(0), enc.shape[0], wk,
                                                wv, bv),
                "set_cross_proj")

    def capture_cross_heads(self, layer, q, selected, n_selected, row_offset, out, lse=None):
        """capture_cross_attention_heads (crates/whisper/src/decoder.rs:796-828).

        ``selected`` lists this layer's (slot, head) pairs; ``q`` is the
        layer's [n_tokens][d_model] float32 query tensor and ``out`` the float32
        capture buffer laid out [row][slot][n_audio] (decoder.rs:821-822).
        With ``lse`` (from ``prefill_cross(..., lse=...)`` on the same rows and
        layer) the capture is one launch instead of two.
        """
        n = len(selected)
        slots = (ctypes.c_size_t * max(n, 1))(*[s for s, _ in selected])
        heads = (ctypes.c_size_t * max(n, 1))(*[h for _, h in selected])
        if lse is None:
            self._c(self._lib.wrs_attn_capture_cross_heads(
                self.ctx.handle, self.handle, layer, q.data_ptr(), q.shape[0], slots, heads, n,
                n_selected, row_offset, out.data_ptr(), out.numel()), "capture_cross_heads")
            return
        self._c(self._lib.wrs_attn_capture_cross_heads_lse(
            self.ctx.handle, self.handle, layer, q.data_ptr(), q.shape[0], slots, heads, n,
            n_selected, row_offset, out.data_ptr(), out.numel(), lse.data_ptr()),
            "capture_cross_heads_lse")
