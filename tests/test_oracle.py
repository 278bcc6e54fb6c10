"""Pins the CPU oracle before anything is compared against it.

Each test names the reference test or the mathematical fact it ports. The
known-answer tests are those of crates/tensor/tests/test_flash_attention_tiled.rs
(same xorshift32 inputs, seeds, shapes and 1e-5 bound) and
crates/tensor/tests/test_flash_attention.rs (modular inputs, 1e-4); the
comparison side is the materialized softmax in float64 (tests/refmath.py).
"""
from __future__ import annotations

import numpy as np
import pytest

from refmath import attention_f64

Q_TILE = 128
KV_TILE = 128


def _py_xorshift(seed, n):
    """Independent pure-Python xorshift32 (test_flash_attention_tiled.rs:22-30)."""
    x = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        out[i] = (np.float32(x) / np.float32(4294967295.0)) * np.float32(2.0) - np.float32(1.0)
    return out


def test_xorshift_matches_independent_python(orc):
    rng = orc.Rng(0x1234_5678)
    a = rng.fill(300)
    b = rng.fill(5)
    ref = _py_xorshift(0x1234_5678, 305)
    np.testing.assert_array_equal(np.concatenate([a, b]), ref)
    assert a.min() >= -1.0 and a.max() < 1.0


def _kat_inputs(orc, t_q, t_kv, n_heads, d_head):
    # seed rule of test_flash_attention_tiled.rs:95
    d_model = n_heads * d_head
    rng = orc.Rng(0x1234_5678 ^ ((t_q << 16) & 0xFFFFFFFF) ^ t_kv)
    return d_model, rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)


def _max_abs_error(orc, t_q, t_kv, n_heads, d_head, causal):
    d_model, q, k, v = _kat_inputs(orc, t_q, t_kv, n_heads, d_head)
    out = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, causal, out)
    ref = attention_f64(q, k, v, t_q, t_kv, n_heads, d_model, causal)
    return float(np.abs(out.reshape(t_q, d_model) - ref).max())


# test_flash_attention_tiled.rs:132-184 (shape list, 1e-5 bound at :126)
KAT_SHAPES = [
    (100, 137, 3, 64, False),
    (100, 137, 3, 64, True),
    (37, 91, 2, 80, False),
    (37, 91, 2, 80, True),
    (Q_TILE + 1, KV_TILE + 1, 2, 64, False),
    (2 * Q_TILE + 3, 2 * KV_TILE + 5, 4, 64, False),
    (Q_TILE + 1, KV_TILE + 1, 2, 64, True),
    (2 * Q_TILE + 3, 2 * KV_TILE + 5, 4, 64, True),
    (90, 33, 3, 64, True),
    (Q_TILE + 40, 37, 3, 64, True),
    (1, 257, 4, 64, False),
    (1, 193, 2, 80, False),
]


@pytest.mark.parametrize("t_q,t_kv,h,dh,causal", KAT_SHAPES)
def test_tiled_kat(orc, t_q, t_kv, h, dh, causal):
    assert _max_abs_error(orc, t_q, t_kv, h, dh, causal) <= 1e-5


def test_single_query_causal_only_sees_first_key(orc):
    # test_flash_attention_tiled.rs:186-205
    d_model, t_kv = 64, 17
    rng = orc.Rng(0xFEED_FACE)
    q, k, v = rng.fill(d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.zeros(d_model, np.float32)
    orc.flash_attention_2(q, k, v, 1, t_kv, 1, d_model, True, out)
    assert np.all(np.abs(out - v[:d_model]) <= 1e-6)


def test_multi_head_attention_kat(orc):
    # test_flash_attention_tiled.rs:207-241
    t_q, t_kv, n_heads, d_head = 48, 70, 5, 64
    d_model = n_heads * d_head
    rng = orc.Rng(0x0BAD_C0DE)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.zeros(t_q * d_model, np.float32)
    orc.multi_head_attention(q, k, v, t_q, t_kv, n_heads, d_model, False, out)
    ref = attention_f64(q, k, v, t_q, t_kv, n_heads, d_model)
    assert np.abs(out.reshape(t_q, d_model) - ref).max() <= 1e-5


def test_stale_output_is_overwritten(orc):
    # test_flash_attention_tiled.rs:243-262
    t_q, t_kv, n_heads, d_head = 40, 100, 2, 64
    d_model = n_heads * d_head
    rng = orc.Rng(0xDEAD_BEEF)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.full(t_q * d_model, np.nan, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, True, out)
    assert np.all(np.isfinite(out))


def _modular_inputs(t_q, t_kv, d_model):
    # test_flash_attention.rs:10-23
    q = ((np.arange(t_q * d_model) % 17).astype(np.float32) - 8.0) * np.float32(0.1)
    k = ((np.arange(t_kv * d_model) % 19).astype(np.float32) - 9.0) * np.float32(0.1)
    v = ((np.arange(t_kv * d_model) % 23).astype(np.float32) - 11.0) * np.float32(0.1)
    return q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_matches_standard(orc, causal):
    # test_flash_attention.rs:3-98: t_q=64, t_kv=128, 4 heads, d_model 64 (d_head 16), 1e-4
    t_q, t_kv, n_heads, d_model = 64, 128, 4, 64
    q, k, v = _modular_inputs(t_q, t_kv, d_model)
    out = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, causal, out)
    ref = attention_f64(q, k, v, t_q, t_kv, n_heads, d_model, causal)
    assert np.abs(out.reshape(t_q, d_model) - ref).max() <= 1e-4


@pytest.mark.parametrize("t_q,t_kv", [(1500, 1500), (64, 1500)])
def test_bench_shapes(orc, t_q, t_kv):
    # bench_flash_attention_tiled.rs:19-25, :142-147, bound 1e-4 at :258-260
    n_heads, d_head = 6, 64
    d_model = n_heads * d_head
    rng = orc.Rng(0x5EED_1234)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, False, out)
    ref = attention_f64(q, k, v, t_q, t_kv, n_heads, d_model)
    assert np.abs(out.reshape(t_q, d_model) - ref).max() <= 1e-4


@pytest.mark.parametrize("t_q,t_kv", [(1500, 1500), (64, 1500), (4096, 4096)])
def test_materialized_baseline_matches_tiled(orc, t_q, t_kv):
    # bench_flash_attention_tiled.rs:142-147 and :258-260: the tiled kernel and
    # the materialized baseline agree within 1e-4 on every benchmark shape
    # (6 heads, d_head 64, one xorshift stream seeded 0x5eed_1234 for q, k, v).
    n_heads, d_head = 6, 64
    d_model = n_heads * d_head
    rng = orc.Rng(0x5EED_1234)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    tiled = np.zeros(t_q * d_model, np.float32)
    mat = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, False, tiled)
    orc.materialized_attention(q, k, v, t_q, t_kv, n_heads, d_model, mat)
    assert np.abs(tiled - mat).max() <= 1e-4
    if t_q * t_kv <= 1500 * 1500:
        ref = attention_f64(q, k, v, t_q, t_kv, n_heads, d_model).ravel()
        assert np.abs(mat - ref).max() <= 1e-5


# ---- edge cases fixed by attention.rs itself -------------------------------

def test_t_q_zero_is_noop(orc):
    out = np.full(0, 7.0, np.float32)
    k = np.ones(5 * 64, np.float32)
    orc.flash_attention_2(np.zeros(0, np.float32), k, k, 0, 5, 1, 64, False, out)


def test_t_kv_zero_zero_fills(orc):
    out = np.full(3 * 64, np.nan, np.float32)
    e = np.zeros(0, np.float32)
    orc.flash_attention_2(np.ones(3 * 64, np.float32), e, e, 3, 0, 1, 64, False, out)
    assert np.all(out == 0.0)


def test_shape_asserts_raise(orc):
    q = np.zeros(64, np.float32)
    with pytest.raises(AssertionError):
        orc.flash_attention_2(q, q, q, 1, 1, 0, 64, False, q.copy())
    with pytest.raises(AssertionError):
        orc.flash_attention_2(q, q, q, 1, 1, 3, 64, False, q.copy())
    with pytest.raises(AssertionError):
        orc.flash_attention_2(q, q, q, 2, 1, 1, 64, False, q.copy())


# ---- closed forms and invariants --------------------------------------------

@pytest.mark.parametrize("t_q", [1, 70])
def test_zero_keys_give_mean_of_values(orc, t_q):
    # K == 0 -> every score 0 -> uniform weights -> mean of V rows
    n_heads, d_head, t_kv = 3, 64, 300
    d_model = n_heads * d_head
    rng = orc.Rng(77)
    q = rng.fill(t_q * d_model)
    k = np.zeros(t_kv * d_model, np.float32)
    v = rng.fill(t_kv * d_model)
    out = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, False, out)
    mean = v.reshape(t_kv, d_model).astype(np.float64).mean(axis=0)
    assert np.abs(out.reshape(t_q, d_model) - mean[None, :]).max() <= 2e-6


@pytest.mark.parametrize("t_q", [1, 50])
def test_dominant_key_selects_its_value(orc, t_q):
    n_heads, d_head, t_kv = 2, 64, 257
    d_model = n_heads * d_head
    rng = orc.Rng(99)
    q = np.ones(t_q * d_model, np.float32)
    k = rng.fill(t_kv * d_model) * np.float32(0.01)
    star = 201
    k.reshape(t_kv, d_model)[star, :] = 4.0  # score 4*64/8 = 32 above the rest
    v = rng.fill(t_kv * d_model)
    out = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, False, out)
    want = v.reshape(t_kv, d_model)[star]
    assert np.abs(out.reshape(t_q, d_model) - want[None, :]).max() <= 1e-5


def test_key_permutation_invariance(orc):
    t_q, t_kv, n_heads, d_head = 33, 300, 2, 64
    d_model = n_heads * d_head
    rng = orc.Rng(5)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    perm = np.random.default_rng(0).permutation(t_kv)
    kp = np.ascontiguousarray(k.reshape(t_kv, d_model)[perm]).ravel()
    vp = np.ascontiguousarray(v.reshape(t_kv, d_model)[perm]).ravel()
    a = np.zeros(t_q * d_model, np.float32)
    b = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, False, a)
    orc.flash_attention_2(q, kp, vp, t_q, t_kv, n_heads, d_model, False, b)
    assert np.abs(a - b).max() <= 1e-6


# ---- softmax_inplace (softmax.rs) -------------------------------------------

def test_softmax_closed_forms(orc):
    x = np.full(37, 3.25, np.float32)
    orc.softmax_inplace(x)
    assert np.abs(x - 1.0 / 37).max() <= 1e-7
    y = np.array([0.0, 200.0, 0.0], np.float32)  # one-hot limit
    orc.softmax_inplace(y)
    assert y[1] == 1.0 and y[0] == 0.0
    e = np.zeros(0, np.float32)
    orc.softmax_inplace(e)  # empty slice is a no-op (softmax.rs:2-4)


def test_softmax_matches_f64_and_shift_invariance(orc):
    rng = np.random.default_rng(3)
    x = rng.normal(size=1500).astype(np.float32) * 3
    a = x.copy()
    orc.softmax_inplace(a)
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    assert np.abs(a - ref).max() <= 1e-7
    assert abs(float(a.astype(np.float64).sum()) - 1.0) <= 1e-5
    b = (x + np.float32(8.0)).astype(np.float32)  # exact shift for these magnitudes
    orc.softmax_inplace(b)
    assert np.abs(a - b).max() <= 1e-7


# ---- dot_f32 (simd.rs) -------------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 7, 8, 31, 32, 64, 80, 100])
def test_dot_exact_on_integers(orc, n):
    a = (np.arange(n) % 7 - 3).astype(np.float32)
    b = (np.arange(n) % 5 - 2).astype(np.float32)
    assert orc.dot_f32(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))


def test_dot_scalar_and_avx2_agree_with_f64(orc):
    rng = np.random.default_rng(11)
    a = rng.normal(size=64).astype(np.float32)
    b = rng.normal(size=64).astype(np.float32)
    ref = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    fast = orc.dot_f32(a, b)
    orc.force_scalar(True)
    try:
        slow = orc.dot_f32(a, b)
    finally:
        orc.force_scalar(False)
    assert abs(fast - ref) <= 1e-5 and abs(slow - ref) <= 1e-5


# ---- single_token_mha_d64 (attention.rs:246-434) ----------------------------

@pytest.mark.parametrize("t_kv", [1, 17, 224, 1500, 1501])
def test_single_token_against_f64(orc, t_kv):
    n_heads, d_model = 5, 5 * 64
    rng = orc.Rng(0xC0FFEE ^ t_kv)
    q, k, v = rng.fill(d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.zeros(d_model, np.float32)
    orc.single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, out)
    ref = attention_f64(q, k, v, 1, t_kv, n_heads, d_model)
    assert np.abs(out - ref.ravel()).max() <= 1e-5
    orc.force_scalar(True)
    try:
        out2 = np.full(d_model, np.nan, np.float32)
        orc.single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, out2)
    finally:
        orc.force_scalar(False)
    assert np.abs(out - out2).max() <= 1e-6


def test_single_token_skips_tiny_weights(orc):
    # attention.rs:366 -- weights below 1e-7 do not reach the output. One key
    # gets weight ~e^-20 (~2e-9) and a value of 1e4, so keeping it would add
    # ~2e-5 to the output.
    d_model, t_kv = 64, 3
    q = np.full(d_model, 1.0, np.float32)
    k = np.zeros((t_kv, d_model), np.float32)
    k[1, :] = -20.0 / 8.0  # score = 64 * (-2.5) * 0.125 = -20
    v = np.zeros((t_kv, d_model), np.float32)
    v[1, :] = 1e4
    out = np.zeros(d_model, np.float32)
    orc.single_token_mha_d64(q, k.ravel(), v.ravel(), t_kv, 1, d_model, out)
    kept = attention_f64(q, k, v, 1, t_kv, 1, d_model)
    skipped = attention_f64(q, k, v, 1, t_kv, 1, d_model, skip_below=1e-7)
    assert np.abs(out - skipped.ravel()).max() <= 1e-7
    assert np.abs(out - kept.ravel()).max() > 1e-5


# ---- multi_head_attention_with_cache (decoder.rs:835-892) ------------------

@pytest.mark.parametrize("n_tokens,t_past,d_head", [(1, 0, 64), (1, 223, 64), (5, 7, 64),
                                                      (4, 30, 80), (1, 9, 80)])
def test_mha_with_cache_against_f64(orc, n_tokens, t_past, d_head):
    n_heads = 3
    d_model = n_heads * d_head
    total = t_past + n_tokens
    rng = orc.Rng(0xABCD ^ total)
    q, k, v = rng.fill(n_tokens * d_model), rng.fill(total * d_model), rng.fill(total * d_model)
    out = np.zeros(n_tokens * d_model, np.float32)
    orc.mha_with_cache(q, k, v, n_tokens, total, t_past, n_heads, d_model, out)
    ref = attention_f64(q, k, v, n_tokens, total, n_heads, d_model, causal=True, q_offset=t_past)
    assert np.abs(out.reshape(n_tokens, d_model) - ref).max() <= 1e-5


def test_mha_with_cache_single_token_dispatch(orc):
    # decoder.rs:852-855: n_tokens == 1 and d_head == 64 -> single_token_mha_d64
    n_heads, d_model, t_past = 4, 256, 40
    rng = orc.Rng(1234)
    q = rng.fill(d_model)
    k, v = rng.fill((t_past + 1) * d_model), rng.fill((t_past + 1) * d_model)
    a = np.zeros(d_model, np.float32)
    b = np.zeros(d_model, np.float32)
    orc.mha_with_cache(q, k, v, 1, t_past + 1, t_past, n_heads, d_model, a)
    orc.single_token_mha_d64(q, k, v, t_past + 1, n_heads, d_model, b)
    np.testing.assert_array_equal(a, b)


# ---- capture_cross_attention_heads (crates/whisper/src/decoder.rs:796-828) ----

def _capture_f64(q, k, n_tokens, n_audio, n_heads, d_model, head):
    dh = d_model // n_heads
    qh = q.reshape(n_tokens, d_model)[:, head * dh:(head + 1) * dh].astype(np.float64)
    kh = k.reshape(n_audio, d_model)[:, head * dh:(head + 1) * dh].astype(np.float64)
    s = qh @ kh.T / np.sqrt(dh)
    e = np.exp(s - s.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("n_audio", [1, 37, 1500])
def test_capture_against_f64_and_layout(orc, n_audio):
    n_tokens, H, dm, n_sel, row_off = 3, 4, 256, 3, 2
    rng = np.random.default_rng(n_audio)
    q = rng.standard_normal(n_tokens * dm).astype(np.float32)
    k = rng.standard_normal(n_audio * dm).astype(np.float32)
    selected = [(2, 1), (0, 3)]  # (slot, head); slot 1 belongs to another layer
    out = np.full((row_off + n_tokens) * n_sel * n_audio, np.nan, np.float32)
    orc.capture_cross_attention_heads(q, k, n_tokens, n_audio, H, dm, selected, n_sel, row_off,
                                      out)
    o = out.reshape(row_off + n_tokens, n_sel, n_audio)
    for slot, head in selected:
        ref = _capture_f64(q, k, n_tokens, n_audio, H, dm, head)
        assert np.abs(o[row_off:, slot] - ref).max() <= 1e-6
    # rows before row_offset and the slot of no pair stay untouched (decoder.rs:821)
    assert np.isnan(o[:row_off]).all() and np.isnan(o[:, 1]).all()


def test_capture_rows_are_distributions(orc):
    """crates/whisper/tests/test_dtw_alignment.rs:60-74: finite, >= 0, rows sum to 1 +- 1e-4."""
    n_tokens, n_audio, H, dm = 5, 1500, 6, 384  # tiny.en width
    rng = np.random.default_rng(7)
    q = (3.0 * rng.standard_normal(n_tokens * dm)).astype(np.float32)
    k = rng.standard_normal(n_audio * dm).astype(np.float32)
    selected = list(enumerate([1, 2, 3, 5]))
    out = np.zeros(n_tokens * len(selected) * n_audio, np.float32)
    orc.capture_cross_attention_heads(q, k, n_tokens, n_audio, H, dm, selected, len(selected), 0,
                                      out)
    assert np.isfinite(out).all() and (out >= 0).all()
    sums = out.reshape(-1, n_audio).astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-4


def test_capture_zero_keys_are_uniform(orc):
    """K == 0: every score is 0, exp(0) = 1, the sum is n exactly, weight = fl(1/n)."""
    n_tokens, n_audio, H, dm = 2, 1500, 2, 128
    q = np.random.default_rng(1).standard_normal(n_tokens * dm).astype(np.float32)
    k = np.zeros(n_audio * dm, np.float32)
    out = np.zeros(n_tokens * n_audio, np.float32)
    orc.capture_cross_attention_heads(q, k, n_tokens, n_audio, H, dm, [(0, 1)], 1, 0, out)
    assert (out == np.float32(1.0) / np.float32(n_audio)).all()


def test_capture_dominant_key(orc):
    """One key aligned with q at a large margin takes all the weight."""
    n_audio, H, dm = 300, 4, 256
    rng = np.random.default_rng(2)
    q = rng.standard_normal(dm).astype(np.float32)
    k = (0.01 * rng.standard_normal(n_audio * dm)).astype(np.float32).reshape(n_audio, dm)
    k[123, 64:128] = 40.0 * q[64:128] / np.linalg.norm(q[64:128])
    out = np.zeros(n_audio, np.float32)
    orc.capture_cross_attention_heads(q, k.ravel().copy(), 1, n_audio, H, dm, [(0, 1)], 1, 0, out)
    assert out.argmax() == 123 and out[123] > 0.999


def test_capture_weights_reproduce_attention(orc):
    """Weights of head h times V[:, h] equal multi_head_attention's head-h output
    (attention.rs:29-41, pinned above): ties the scale and head offset to it."""
    n_tokens, n_audio, H, dm = 4, 211, 4, 256
    rng = np.random.default_rng(3)
    q = rng.standard_normal(n_tokens * dm).astype(np.float32)
    k = rng.standard_normal(n_audio * dm).astype(np.float32)
    v = rng.standard_normal(n_audio * dm).astype(np.float32)
    att = np.zeros(n_tokens * dm, np.float32)
    orc.multi_head_attention(q, k, v, n_tokens, n_audio, H, dm, False, att)
    selected = [(h, h) for h in range(H)]
    out = np.zeros(n_tokens * H * n_audio, np.float32)
    orc.capture_cross_attention_heads(q, k, n_tokens, n_audio, H, dm, selected, H, 0, out)
    w = out.reshape(n_tokens, H, n_audio).astype(np.float64)
    vv = v.reshape(n_audio, H, 64).astype(np.float64)
    got = np.einsum("thj,jhd->thd", w, vv).reshape(n_tokens, dm)
    assert np.abs(got - att.reshape(n_tokens, dm)).max() <= 1e-5


def test_capture_empty_audio_is_noop(orc):
    out = np.full(6, 7.0, np.float32)
    orc.capture_cross_attention_heads(np.ones(128, np.float32), np.zeros(0, np.float32), 1, 0, 2,
                                      128, [(0, 0)], 1, 0, out)
    assert (out == 7.0).all()


# ---- f16_linear / dot_f16_f32 (crates/tensor/src/ops/quant.rs:415-473, simd.rs:593-700) ----

def test_f16_to_f32_all_bit_patterns(orc):
    """Every binary16 pattern widens exactly (numpy's conversion is IEEE exact)."""
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("n", [0, 1, 3, 8, 31, 32, 40, 64, 100, 1280])
def test_dot_f16_exact_on_integers(orc, n):
    rng = np.random.default_rng(n)
    w = rng.integers(-8, 9, n).astype(np.float16)
    x = rng.integers(-8, 9, n).astype(np.float32)
    assert orc.dot_f16_f32(w, x) == float(np.dot(w.astype(np.float64), x.astype(np.float64)))


def test_dot_f16_scalar_and_avx2_agree_with_f64(orc):
    rng = np.random.default_rng(5)
    for n in (7, 33, 64, 391, 1280):
        w = rng.standard_normal(n).astype(np.float16)
        x = rng.standard_normal(n).astype(np.float32)
        exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        bound = n * 2.0 ** -23 * float(np.abs(w.astype(np.float64) * x).sum())
        vec = orc.dot_f16_f32(w, x)
        orc.lib().wrs_oracle_force_scalar(1)
        try:
            sca = orc.dot_f16_f32(w, x)
        finally:
            orc.lib().wrs_oracle_force_scalar(0)
        assert abs(vec - exact) <= bound and abs(sca - exact) <= bound


def test_f16_linear_against_f64_layout_and_bias(orc):
    rows, cols, T = 96, 320, 7
    rng = np.random.default_rng(9)
    w = (0.05 * rng.standard_normal((rows, cols))).astype(np.float16)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    b = rng.standard_normal(rows).astype(np.float32)
    out = np.full(T * rows, np.nan, np.float32)
    orc.f16_linear(w, rows, cols, x.ravel(), b, T, out)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b  # [T][rows] = output[t*rows + r]
    absw = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert (np.abs(out.reshape(T, rows) - ref) <= cols * 2.0 ** -23 * absw + 1e-6).all()
    # no bias: the plain dot (quant.rs:464-467)
    out2 = np.zeros(T * rows, np.float32)
    orc.f16_linear(w, rows, cols, x.ravel(), None, T, out2)
    assert np.array_equal(out2.reshape(T, rows) + b, out.reshape(T, rows))  # fl(dot + b)


def test_f16_linear_identity_and_single_token(orc):
    """W = I copies x exactly; the single-token branch (quant.rs:434-437) gives
    the same numbers as one row of the multi-token branch."""
    n = 64
    x = np.random.default_rng(3).standard_normal((3, n)).astype(np.float32)
    out = np.zeros(3 * n, np.float32)
    orc.f16_linear(np.eye(n, dtype=np.float16), n, n, x.ravel(), None, 3, out)
    assert np.array_equal(out, x.ravel())
    w = np.random.default_rng(4).standard_normal((40, n)).astype(np.float16)
    many = np.zeros(3 * 40, np.float32)
    orc.f16_linear(w, 40, n, x.ravel(), None, 3, many)
    one = np.zeros(40, np.float32)
    orc.f16_linear(w, 40, n, x[1].copy(), None, 1, one)
    assert np.array_equal(one, many.reshape(3, 40)[1])


def test_f16_linear_asserts(orc):
    w = np.zeros((4, 8), np.float16)
    with pytest.raises(AssertionError):
        orc.f16_linear(w, 4, 8, np.zeros(15, np.float32), None, 2, np.zeros(8, np.float32))


# ---- layer_norm (crates/tensor/src/ops/norm.rs) and gelu (crates/tensor/src/ops/gelu.rs) ----

def _ln_f64(x, g, b, eps):
    x = x.astype(np.float64)
    m = x.mean(axis=-1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


@pytest.mark.parametrize("d", [1, 7, 64, 384, 1280, 1283])
def test_layer_norm_against_f64(orc, d):
    rng = np.random.default_rng(d)
    T = 6
    x = (3.0 * rng.standard_normal((T, d)) + 1.5).astype(np.float32)
    g = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    out = np.zeros(T * d, np.float32)
    orc.layer_norm(x.ravel(), g, b, 1e-5, T, d, out)
    ref = _ln_f64(x, g, b, 1e-5)
    assert np.abs(out.reshape(T, d) - ref).max() <= 2e-5 * max(1.0, np.abs(ref).max())
    orc.lib().wrs_oracle_force_scalar(1)
    try:
        out2 = np.zeros(T * d, np.float32)
        orc.layer_norm(x.ravel(), g, b, 1e-5, T, d, out2)
    finally:
        orc.lib().wrs_oracle_force_scalar(0)
    assert np.abs(out2.reshape(T, d) - ref).max() <= 2e-5 * max(1.0, np.abs(ref).max())


def test_layer_norm_closed_forms(orc):
    d = 256
    g = np.random.default_rng(1).standard_normal(d).astype(np.float32)
    b = np.random.default_rng(2).standard_normal(d).astype(np.float32)
    # a constant row has zero variance: the output is beta exactly
    x = np.full((1, d), 3.25, np.float32)
    out = np.zeros(d, np.float32)
    orc.layer_norm(x.ravel(), g, b, 1e-5, 1, d, out)
    assert np.array_equal(out, b)
    # gamma = 1, beta = 0: mean 0 and variance v / (v + eps) of the output
    x = np.random.default_rng(3).standard_normal((4, d)).astype(np.float32)
    out = np.zeros(4 * d, np.float32)
    orc.layer_norm(x.ravel(), np.ones(d, np.float32), np.zeros(d, np.float32), 1e-5, 4, d, out)
    o = out.reshape(4, d).astype(np.float64)
    v = x.astype(np.float64).var(axis=1)
    assert np.abs(o.mean(axis=1)).max() < 1e-6
    assert np.abs(o.var(axis=1) - v / (v + 1e-5)).max() < 1e-5


def test_layer_norm_asserts(orc):
    with pytest.raises(AssertionError):
        orc.layer_norm(np.zeros(10, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32),
                       1e-5, 2, 4, np.zeros(8, np.float32))


def test_gelu_against_f64_and_closed_forms(orc):
    x = np.linspace(-12, 12, 20001).astype(np.float32)
    y = x.copy()
    orc.gelu_inplace(y)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(0.7978846 * xd * (1 + 0.044715 * xd * xd)))
    assert np.abs(y - ref).max() <= 4e-7 * np.maximum(1.0, np.abs(ref)).max()
    assert orc.gelu(0.0) == 0.0
    # tanh-form identity: gelu(x) - gelu(-x) = x
    assert np.abs((y - y[::-1]) - x).max() <= 2e-6 * 12
    # large |x|: identity and zero
    assert orc.gelu(30.0) == 30.0 and orc.gelu(-30.0) == 0.0
