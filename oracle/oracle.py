"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

The oracle is a C restatement of the reference's CPU attention path
(crates/tensor/src/ops/attention.rs, crates/tensor/src/ops/softmax.rs,
crates/tensor/src/simd.rs:4-119 and :593-700, crates/tensor/src/ops/quant.rs:343-473,
crates/whisper/src/decoder.rs:796-892).
Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this module, and only as the parity reference or the timed CPU baseline. The
product package (``whisper.rs_amd``) never imports it.

Function names and argument meaning follow the reference; shape violations
that the reference turns into a panic (``assert!`` / ``assert_eq!``, e.g.
crates/tensor/src/ops/attention.rs:79-88) raise ``AssertionError`` here.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "build" / "liboracle.so"
_lib = None

Q_TILE = 128  # crates/tensor/src/ops/attention.rs:13
KV_TILE = 128  # crates/tensor/src/ops/attention.rs:26

_f32p = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def build() -> None:
    """Compile the oracle with oracle/Makefile (gcc)."""
    import subprocess

    subprocess.run(["make", "-B", "-C", str(_HERE)], check=True,
                   stdout=subprocess.DEVNULL)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {_LIB_PATH}; run oracle/Makefile")
        L = ctypes.CDLL(str(_LIB_PATH))
        L.wrs_oracle_softmax_inplace.argtypes = [_f32p, _sz]
        L.wrs_oracle_softmax_inplace.restype = None
        L.wrs_oracle_dot_f32.argtypes = [_f32p, _f32p, _sz]
        L.wrs_oracle_dot_f32.restype = ctypes.c_float
        for name in ("wrs_oracle_flash_attention_2", "wrs_oracle_multi_head_attention"):
            fn = getattr(L, name)
            fn.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, ctypes.c_int, _f32p,
                           ctypes.c_int]
            fn.restype = ctypes.c_int
        L.wrs_oracle_materialized_attention.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz,
                                                        _f32p, ctypes.c_int]
        L.wrs_oracle_materialized_attention.restype = ctypes.c_int
        L.wrs_oracle_single_token_mha_d64.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p]
        L.wrs_oracle_single_token_mha_d64.restype = ctypes.c_int
        L.wrs_oracle_mha_with_cache.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                                _f32p]
        L.wrs_oracle_mha_with_cache.restype = ctypes.c_int
        _szp = ctypes.POINTER(_sz)
        L.wrs_oracle_capture_cross_heads.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _sz, _szp, _szp,
                                                     _sz, _sz, _sz, _f32p]
        L.wrs_oracle_capture_cross_heads.restype = ctypes.c_int
        _u16p = ctypes.POINTER(ctypes.c_uint16)
        L.wrs_oracle_dot_f16_f32.argtypes = [_u16p, _f32p, _sz]
        L.wrs_oracle_dot_f16_f32.restype = ctypes.c_float
        L.wrs_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.wrs_oracle_f16_to_f32.restype = ctypes.c_float
        L.wrs_oracle_f16_linear.argtypes = [_u16p, _sz, _sz, _f32p, _f32p, _sz, _f32p,
                                            ctypes.c_int]
        L.wrs_oracle_f16_linear.restype = ctypes.c_int
        L.wrs_oracle_layer_norm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_float, _sz, _sz, _f32p]
        L.wrs_oracle_layer_norm.restype = ctypes.c_int
        L.wrs_oracle_gelu.argtypes = [ctypes.c_float]
        L.wrs_oracle_gelu.restype = ctypes.c_float
        L.wrs_oracle_gelu_inplace.argtypes = [_f32p, _sz]
        L.wrs_oracle_gelu_inplace.restype = None
        L.wrs_oracle_xorshift_fill.argtypes = [ctypes.POINTER(ctypes.c_uint32), _f32p, _sz]
        L.wrs_oracle_xorshift_fill.restype = None
        L.wrs_oracle_uses_avx2.argtypes = []
        L.wrs_oracle_uses_avx2.restype = ctypes.c_int
        L.wrs_oracle_force_scalar.argtypes = [ctypes.c_int]
        L.wrs_oracle_force_scalar.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise AssertionError(f"{what}: reference would panic (code {rc})")


class Rng:
    """xorshift32 of crates/tensor/tests/test_flash_attention_tiled.rs:15-35."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint32(seed & 0xFFFFFFFF)

    def fill(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().wrs_oracle_xorshift_fill(ctypes.byref(self.state), _ptr(out), n)
        return out


def softmax_inplace(x: np.ndarray) -> None:
    lib().wrs_oracle_softmax_inplace(_ptr(x), x.size)


def dot_f32(a: np.ndarray, b: np.ndarray) -> float:
    assert a.size == b.size  # simd.rs:5
    return float(lib().wrs_oracle_dot_f32(_ptr(a), _ptr(b), a.size))


def _threads(n_threads):
    if n_threads is None:
        return int(os.environ.get("WRS_ORACLE_THREADS", "0"))
    return n_threads


def flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, causal, output, n_threads=None):
    """crates/tensor/src/ops/attention.rs:68-243."""
    assert n_heads > 0, "n_heads must be non-zero"
    assert d_model % n_heads == 0
    assert q.size == t_q * d_model and k.size == t_kv * d_model
    assert v.size == t_kv * d_model and output.size == t_q * d_model
    rc = lib().wrs_oracle_flash_attention_2(_ptr(q), _ptr(k), _ptr(v), t_q, t_kv, n_heads,
                                            d_model, int(bool(causal)), _ptr(output),
                                            _threads(n_threads))
    _check(rc, "flash_attention_2")


def materialized_attention(q, k, v, t_q, t_kv, n_heads, d_model, output, n_threads=None):
    """crates/tensor/tests/bench_flash_attention_tiled.rs:46-107: full score
    matrix per head, softmax_inplace per row, then scores x V (the reference's
    benchmark baseline)."""
    assert n_heads > 0 and d_model % n_heads == 0
    assert q.size == t_q * d_model and k.size == t_kv * d_model
    assert v.size == t_kv * d_model and output.size == t_q * d_model
    rc = lib().wrs_oracle_materialized_attention(_ptr(q), _ptr(k), _ptr(v), t_q, t_kv, n_heads,
                                                 d_model, _ptr(output), _threads(n_threads))
    _check(rc, "materialized_attention")


def multi_head_attention(q, k, v, t_q, t_kv, n_heads, d_model, causal, output, n_threads=None):
    """crates/tensor/src/ops/attention.rs:29-41."""
    assert n_heads > 0, "n_heads must be non-zero"
    assert d_model % n_heads == 0
    assert q.size == t_q * d_model and k.size == t_kv * d_model
    assert v.size == t_kv * d_model and output.size == t_q * d_model
    rc = lib().wrs_oracle_multi_head_attention(_ptr(q), _ptr(k), _ptr(v), t_q, t_kv, n_heads,
                                               d_model, int(bool(causal)), _ptr(output),
                                               _threads(n_threads))
    _check(rc, "multi_head_attention")


def single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, output):
    """crates/tensor/src/ops/attention.rs:246-274."""
    rc = lib().wrs_oracle_single_token_mha_d64(_ptr(q), _ptr(k), _ptr(v), t_kv, n_heads,
                                               d_model, _ptr(output))
    _check(rc, "single_token_mha_d64")


def mha_with_cache(q, k, v, n_tokens, total_tokens, t_past, n_heads, d_model, output):
    """crates/whisper/src/decoder.rs:835-892 (multi_head_attention_with_cache)."""
    assert q.size == n_tokens * d_model  # decoder.rs:847
    assert k.size == total_tokens * d_model and v.size == total_tokens * d_model
    assert output.size == n_tokens * d_model
    rc = lib().wrs_oracle_mha_with_cache(_ptr(q), _ptr(k), _ptr(v), n_tokens, total_tokens,
                                         t_past, n_heads, d_model, _ptr(output))
    _check(rc, "multi_head_attention_with_cache")


def capture_cross_attention_heads(q, k, n_tokens, n_audio, n_heads, d_model, selected,
                                  n_selected, row_offset, out):
    """crates/whisper/src/decoder.rs:796-828; ``selected`` is [(slot, head), ...]."""
    assert n_heads > 0 and d_model % n_heads == 0
    assert q.size >= n_tokens * d_model and k.size >= n_audio * d_model
    assert out.size >= (row_offset + n_tokens) * n_selected * n_audio  # decoder.rs:812
    d_head = d_model // n_heads
    for slot, head in selected:
        assert (head + 1) * d_head <= d_model  # the q/k slices of decoder.rs:815-817
        assert ((row_offset + n_tokens - 1) * n_selected + slot + 1) * n_audio <= out.size or \
            n_tokens == 0
    n = len(selected)
    slots = (ctypes.c_size_t * max(n, 1))(*[s for s, _ in selected])
    heads = (ctypes.c_size_t * max(n, 1))(*[h for _, h in selected])
    rc = lib().wrs_oracle_capture_cross_heads(_ptr(q), _ptr(k), n_tokens, n_audio, n_heads,
                                              d_model, slots, heads, n, n_selected, row_offset,
                                              _ptr(out))
    _check(rc, "capture_cross_attention_heads")


def _u16(a: np.ndarray):
    assert a.dtype == np.float16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def f16_to_f32(bits: int) -> float:
    return float(lib().wrs_oracle_f16_to_f32(bits))


def dot_f16_f32(w: np.ndarray, x: np.ndarray) -> float:
    """crates/tensor/src/simd.rs:593-700; w is float16 (the weight row's halves)."""
    assert w.size == x.size  # simd.rs:594
    return float(lib().wrs_oracle_dot_f16_f32(_u16(w), _ptr(x), x.size))


def f16_linear(w, rows, cols, x, bias, num_tokens, output, n_threads=None):
    """crates/tensor/src/ops/quant.rs:415-473 (LinearWeight::linear, weight.rs:116-137):
    output[t * rows + r] = W[r] . x[t] + bias[r]; w is float16 [rows][cols]."""
    assert x.size == num_tokens * cols  # quant.rs:424
    assert output.size == num_tokens * rows  # quant.rs:425
    if bias is not None:
        assert bias.size == rows  # quant.rs:427
    assert w.size == rows * cols  # quant.rs:440
    rc = lib().wrs_oracle_f16_linear(_u16(w), rows, cols, _ptr(x),
                                     None if bias is None else _ptr(bias), num_tokens,
                                     _ptr(output), _threads(n_threads))
    _check(rc, "f16_linear")


def layer_norm(x, gamma, beta, eps, num_tokens, d_model, out):
    """crates/tensor/src/ops/norm.rs:116-143."""
    assert x.size == num_tokens * d_model and out.size == num_tokens * d_model  # :124-125
    assert gamma.size == d_model and beta.size == d_model  # :126-127
    lib().wrs_oracle_layer_norm(_ptr(x), _ptr(gamma), _ptr(beta), eps, num_tokens, d_model,
                                _ptr(out))


def gelu(x: float) -> float:
    """crates/tensor/src/ops/gelu.rs:6-9."""
    return float(lib().wrs_oracle_gelu(x))


def gelu_inplace(data: np.ndarray) -> None:
    """crates/tensor/src/ops/gelu.rs:11-23."""
    lib().wrs_oracle_gelu_inplace(_ptr(data), data.size)


def uses_avx2() -> bool:
    return bool(lib().wrs_oracle_uses_avx2())


def force_scalar(on: bool) -> None:
    lib().wrs_oracle_force_scalar(int(bool(on)))
