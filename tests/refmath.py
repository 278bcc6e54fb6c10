"""Brute-force float64 attention used to pin the oracle (test helper).

This is the materialized algorithm the reference's own tests compare against
(crates/tensor/tests/test_flash_attention_tiled.rs:41-89,
crates/tensor/tests/test_flash_attention.rs:100-143): full score matrix,
softmax per row, then P @ V -- computed here in float64 so it is independent
of every f32 summation order.
"""
from __future__ import annotations

import numpy as np


def attention_f64(q, k, v, t_q, t_kv, n_heads, d_model, causal=False, q_offset=0,
                  skip_below=None):
    """softmax(QK^T / sqrt(d_head) [+ mask j <= i + q_offset]) V per head.

    Inputs are token-major ``[t][d_model]``; returns float64 ``[t_q][d_model]``.
    ``skip_below`` drops softmax weights below that value before P @ V (the
    decode kernels' rule, crates/tensor/src/ops/attention.rs:366).
    """
    d_head = d_model // n_heads
    q = np.asarray(q, np.float64).reshape(t_q, n_heads, d_head)
    k = np.asarray(k, np.float64).reshape(t_kv, n_heads, d_head)
    v = np.asarray(v, np.float64).reshape(t_kv, n_heads, d_head)
    out = np.zeros((t_q, n_heads, d_head))
    if t_kv == 0:
        return out.reshape(t_q, d_model)
    s = np.einsum("ihd,jhd->hij", q, k) / np.sqrt(d_head)
    if causal:
        i = np.arange(t_q)[:, None] + q_offset
        j = np.arange(t_kv)[None, :]
        s = np.where(j <= i, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    p /= p.sum(axis=-1, keepdims=True)
    if skip_below is not None:
        p = np.where(p < skip_below, 0.0, p)
    out = np.einsum("hij,jhd->ihd", p, v)
    return out.reshape(t_q, d_model)
