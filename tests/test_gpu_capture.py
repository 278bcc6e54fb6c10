"""GPU parity of the DTW alignment-head capture
(capture_cross_attention_heads, crates/whisper/src/decoder.rs:796-828) over the
f16 cross plane of the device KV arena, against the CPU oracle run on the same
f16-rounded keys."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note

pytestmark = pytest.mark.gpu

TOL32 = 1e-5  # f32 weights; keys are exact f16 values on both sides

# dtw.rs AlignmentHeadsPreset::LargeV3 (text layer, head)
LARGE_V3_HEADS = [(7, 0), (10, 17), (12, 18), (13, 12), (16, 1), (17, 14), (19, 11), (21, 4),
                  (24, 1), (25, 6)]


@pytest.fixture(scope="module")
def W(wrs):
    from wrs_amd import workloads
    return workloads


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


def _layer_pairs(heads, layer):
    # decoder.rs:679-687: (slot, head) of every selected head that sits in `layer`
    return [(slot, h) for slot, (l, h) in enumerate(heads) if l == layer]


def _oracle(orc, q, k, n_tokens, n_audio, H, dm, selected, n_sel, row_off, out):
    orc.capture_cross_attention_heads(np.ascontiguousarray(q.ravel()), np.ascontiguousarray(
        k.ravel()), n_tokens, n_audio, H, dm, selected, n_sel, row_off, out)


@pytest.mark.parametrize("n_tokens,n_audio", [(1, 1), (1, 1500), (5, 37), (8, 1500), (9, 1500),
                                              (130, 1500), (3, 2048), (17, 129),
                                              (16, 1500), (33, 1501), (2, 15), (3, 3000)])
def test_capture_matches_oracle(wrs, orc, ctx, W, n_tokens, n_audio):
    note(f"capture n_tokens={n_tokens} n_audio={n_audio}")
    H, dm, n_layers = 4, 256, 2
    arena = wrs.KvArena(n_layers, 1, H, 448, 3000, ctx=ctx)
    ks = [W.normal((n_audio, dm), 100 + l, storage="f16") for l in range(n_layers)]
    for l in range(n_layers):
        arena.set_cross(l, dev(ks[l]), dev(W.normal((n_audio, dm), 110 + l, storage="f16")))
    heads = [(1, 3), (0, 2), (1, 0), (1, 3)]  # the same head twice: two slots
    n_sel, row_off = len(heads), 2
    q = W.normal((n_tokens, dm), 120, sigma=2.0)
    size = (row_off + n_tokens) * n_sel * n_audio
    out = torch.full((size,), float("nan"), device="cuda")
    ref = np.full(size, np.nan, np.float32)
    for layer in range(n_layers):
        sel = _layer_pairs(heads, layer)
        arena.capture_cross_heads(layer, dev(q), sel, n_sel, row_off, out)
        _oracle(orc, q, ks[layer], n_tokens, n_audio, H, dm, sel, n_sel, row_off, ref)
    got = host(out)
    # every written weight matches; the rows before row_offset stay untouched
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.isnan(got.reshape(row_off + n_tokens, -1)[:row_off]).all()
    w = ~np.isnan(ref)
    assert maxerr(got[w], ref[w]) <= TOL32
    arena.close()


def test_capture_large_v3_preset(wrs, orc, ctx, W):
    """whisper-large-v3 geometry (20 heads, d_model 1280, 1500 frames), the
    LargeV3 preset over every selected layer, one segment of 96 tokens."""
    H, dm, n_audio, n_tokens, n_layers = 20, 1280, 1500, 96, 32
    note("capture large-v3 preset")
    arena = wrs.KvArena(n_layers, 1, H, 448, n_audio, ctx=ctx)
    layers = sorted({l for l, _ in LARGE_V3_HEADS})
    ks = {}
    for l in layers:
        ks[l] = W.normal((n_audio, dm), 200 + l, sigma=1.5, storage="f16")
        arena.set_cross(l, dev(ks[l]), dev(np.zeros((n_audio, dm), np.float32)))
    n_sel = len(LARGE_V3_HEADS)
    out = torch.full((n_tokens * n_sel * n_audio,), float("nan"), device="cuda")
    ref = np.full(n_tokens * n_sel * n_audio, np.nan, np.float32)
    for l in layers:
        q = W.normal((n_tokens, dm), 300 + l, sigma=1.5)
        sel = _layer_pairs(LARGE_V3_HEADS, l)
        arena.capture_cross_heads(l, dev(q), sel, n_sel, 0, out)
        _oracle(orc, q, ks[l], n_tokens, n_audio, H, dm, sel, n_sel, 0, ref)
    got = host(out)
    assert not np.isnan(got).any()
    assert maxerr(got, ref) <= TOL32
    # crates/whisper/tests/test_dtw_alignment.rs:60-74 row checks
    assert (got >= 0).all()
    sums = got.reshape(-1, n_audio).astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-4
    arena.close()


def test_capture_all_heads_many_pairs(wrs, orc, ctx, W):
    """40 pairs in one layer (more than one launch's 32), peaked rows."""
    H, dm, n_audio, n_tokens = 20, 1280, 1500, 6
    note("capture 40 pairs")
    arena = wrs.KvArena(1, 1, H, 448, n_audio, ctx=ctx)
    k = W.normal((n_audio, dm), 400, storage="f16")
    arena.set_cross(0, dev(k), dev(k))
    q = W.normal((n_tokens, dm), 401, sigma=6.0)  # scores with std ~6: near one-hot rows
    sel = [(s, (7 * s) % H) for s in range(40)]
    out = torch.full((n_tokens * 40 * n_audio,), float("nan"), device="cuda")
    arena.capture_cross_heads(0, dev(q), sel, 40, 0, out)
    ref = np.zeros(n_tokens * 40 * n_audio, np.float32)
    _oracle(orc, q, k, n_tokens, n_audio, H, dm, sel, 40, 0, ref)
    got = host(out)
    assert maxerr(got, ref) <= TOL32
    assert got.reshape(-1, n_audio).max(axis=1).min() > 0.05  # really peaked
    arena.close()


def test_capture_argument_errors(wrs, ctx, W):
    note("capture argument errors")
    H, dm = 4, 256
    arena = wrs.KvArena(1, 1, H, 448, 100, ctx=ctx)
    k = W.normal((100, dm), 500, storage="f16")
    arena.set_cross(0, dev(k), dev(k))
    q = dev(W.normal((2, dm), 501))
    out = torch.zeros(2 * 2 * 100, device="cuda")
    with pytest.raises(AssertionError):  # head index past n_heads (q/k slice panic)
        arena.capture_cross_heads(0, q, [(0, 4)], 2, 0, out)
    with pytest.raises(AssertionError):  # slot past n_selected
        arena.capture_cross_heads(0, q, [(2, 0)], 2, 0, out)
    with pytest.raises(AssertionError):  # out shorter than (row_offset + n) * n_sel * n_audio
        arena.capture_cross_heads(0, q, [(0, 0)], 2, 1, out)
    with pytest.raises(RuntimeError):  # layer outside the arena
        arena.capture_cross_heads(1, q, [(0, 0)], 2, 0, out)
    # no pairs / no rows: nothing is written
    arena.capture_cross_heads(0, q, [], 2, 0, out)
    arena.capture_cross_heads(0, q[:0], [(0, 0)], 2, 0, out)
    assert float(out.abs().sum()) == 0.0
    arena.close()


# ---- one-pass capture from the attention pass's row statistics -----------------

def _lse_ref(q, k, n_tokens, n_audio, H, dm):
    """float64 (max, sum) per (head, row) in the exp2 domain, s = q.k / 8."""
    ref = np.zeros((H, n_tokens, 2))
    for h in range(H):
        s = (q[:, h * 64:(h + 1) * 64].astype(np.float64) @
             k[:, h * 64:(h + 1) * 64].astype(np.float64).T) * 0.125 * np.log2(np.e)
        m = s.max(axis=1)
        ref[h, :, 0] = m
        ref[h, :, 1] = np.exp2(s - m[:, None]).sum(axis=1)
    return ref


@pytest.mark.parametrize("n_tokens,n_audio", [(1, 1500), (5, 37), (16, 1500), (33, 1501),
                                              (130, 1500), (3, 3000)])
def test_prefill_cross_lse_statistics(wrs, orc, ctx, W, n_tokens, n_audio):
    # the attention output is wrs_attn_prefill_cross's; the statistics are the
    # rows' softmax max and sum (exp2 domain)
    note(f"prefill_cross_lse n_tokens={n_tokens} n_audio={n_audio}")
    H, dm = 4, 256
    arena = wrs.KvArena(1, 1, H, 448, 3000, ctx=ctx)
    k = W.normal((n_audio, dm), 130, storage="f16")
    v = W.normal((n_audio, dm), 131, storage="f16")
    arena.set_cross(0, dev(k), dev(v))
    q = W.normal((n_tokens, dm), 132, sigma=2.0)
    out = torch.full((n_tokens, dm), float("nan"), device="cuda")
    lse = torch.full((2 * H * n_tokens,), float("nan"), device="cuda")
    arena.prefill_cross(0, dev(q), out, lse=lse)
    ref_out = np.zeros(n_tokens * dm, np.float32)
    orc.flash_attention_2(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n_tokens,
                          n_audio, H, dm, False, ref_out)
    assert maxerr(host(out), ref_out.reshape(n_tokens, dm)) <= TOL32
    got = host(lse).reshape(H, n_tokens, 2)
    ref = _lse_ref(q, k, n_tokens, n_audio, H, dm)
    assert np.abs(got[..., 0] - ref[..., 0]).max() <= 1e-5 * max(1.0, np.abs(ref[..., 0]).max())
    assert (np.abs(got[..., 1] - ref[..., 1]) / ref[..., 1]).max() <= 1e-5
    if n_tokens > 1:  # the same kernel as the plain call for prompt rows
        plain = torch.zeros_like(out)
        arena.prefill_cross(0, dev(q), plain)
        assert torch.equal(out, plain)
    arena.close()


@pytest.mark.parametrize("n_tokens,n_audio", [(1, 1500), (5, 37), (16, 1500), (33, 1501),
                                              (130, 1500), (17, 129), (3, 3000)])
def test_capture_one_pass_matches_oracle(wrs, orc, ctx, W, n_tokens, n_audio):
    # decoder.rs:698-721's order: the cross-attention of the rows, then the
    # capture, here one launch on the attention's statistics. The statistics
    # come from other score sums than the capture's exact-product ones, so the
    # bound is the two-pass one plus 1e-5 relative to the weight.
    note(f"one-pass capture n_tokens={n_tokens} n_audio={n_audio}")
    H, dm, n_layers = 4, 256, 2
    arena = wrs.KvArena(n_layers, 1, H, 448, 3000, ctx=ctx)
    ks = [W.normal((n_audio, dm), 140 + l, storage="f16") for l in range(n_layers)]
    for l in range(n_layers):
        arena.set_cross(l, dev(ks[l]), dev(W.normal((n_audio, dm), 150 + l, storage="f16")))
    heads = [(1, 3), (0, 2), (1, 0), (1, 3)]
    n_sel, row_off = len(heads), 2
    q = W.normal((n_tokens, dm), 160, sigma=2.0)
    size = (row_off + n_tokens) * n_sel * n_audio
    out = torch.full((size,), float("nan"), device="cuda")
    two = torch.full((size,), float("nan"), device="cuda")
    ref = np.full(size, np.nan, np.float32)
    att = torch.zeros((n_tokens, dm), device="cuda")
    lse = torch.zeros((2 * H * n_tokens,), device="cuda")
    for layer in range(n_layers):
        sel = _layer_pairs(heads, layer)
        arena.prefill_cross(layer, dev(q), att, lse=lse)
        arena.capture_cross_heads(layer, dev(q), sel, n_sel, row_off, out, lse=lse)
        arena.capture_cross_heads(layer, dev(q), sel, n_sel, row_off, two)
        _oracle(orc, q, ks[layer], n_tokens, n_audio, H, dm, sel, n_sel, row_off, ref)
    got, got2 = host(out), host(two)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    w = ~np.isnan(ref)
    err = np.abs(got[w].astype(np.float64) - ref[w])
    note(f"  max|one-pass - oracle| = {err.max():.3e}, "
         f"max|one-pass - two-pass| = {np.abs(got[w] - got2[w]).max():.3e}")
    assert (err <= TOL32 + 1e-5 * ref[w]).all()
    rows = got[w].reshape(-1, n_audio).astype(np.float64).sum(axis=1)
    assert np.abs(rows - 1.0).max() <= 1e-5
    arena.close()


def test_capture_one_pass_large_v3_preset(wrs, orc, ctx, W):
    """The LargeV3 preset over every selected layer, 96 tokens, one launch per
    layer; the row checks of crates/whisper/tests/test_dtw_alignment.rs:60-74."""
    H, dm, n_audio, n_tokens, n_layers = 20, 1280, 1500, 96, 32
    note("one-pass capture large-v3 preset")
    arena = wrs.KvArena(n_layers, 1, H, 448, n_audio, ctx=ctx)
    layers = sorted({l for l, _ in LARGE_V3_HEADS})
    ks = {}
    for l in layers:
        ks[l] = W.normal((n_audio, dm), 200 + l, sigma=1.5, storage="f16")
        arena.set_cross(l, dev(ks[l]), dev(np.zeros((n_audio, dm), np.float32)))
    n_sel = len(LARGE_V3_HEADS)
    out = torch.full((n_tokens * n_sel * n_audio,), float("nan"), device="cuda")
    ref = np.full(n_tokens * n_sel * n_audio, np.nan, np.float32)
    att = torch.zeros((n_tokens, dm), device="cuda")
    lse = torch.zeros((2 * H * n_tokens,), device="cuda")
    for l in layers:
        q = W.normal((n_tokens, dm), 300 + l, sigma=1.5)
        sel = _layer_pairs(LARGE_V3_HEADS, l)
        arena.prefill_cross(l, dev(q), att, lse=lse)
        arena.capture_cross_heads(l, dev(q), sel, n_sel, 0, out, lse=lse)
        _oracle(orc, q, ks[l], n_tokens, n_audio, H, dm, sel, n_sel, 0, ref)
    got = host(out)
    assert not np.isnan(got).any()
    err = np.abs(got.astype(np.float64) - ref)
    note(f"  max|one-pass - oracle| = {err.max():.3e}")
    assert (err <= TOL32 + 1e-5 * ref).all()
    assert (got >= 0).all()
    sums = got.reshape(-1, n_audio).astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-4
    arena.close()


def test_capture_one_pass_null_statistics_refused(wrs, ctx, W):
    note("one-pass capture without statistics -> error")
    H, dm = 4, 256
    arena = wrs.KvArena(1, 1, H, 448, 100, ctx=ctx)
    k = W.normal((100, dm), 400, storage="f16")
    arena.set_cross(0, dev(k), dev(k))
    q = torch.zeros((2, dm), device="cuda")
    out = torch.zeros((2 * 100,), device="cuda")
    lib = wrs._lib.lib()
    slots = (ctypes.c_size_t * 1)(0)
    heads = (ctypes.c_size_t * 1)(1)
    rc = lib.wrs_attn_capture_cross_heads_lse(ctx.handle, arena.handle, 0, q.data_ptr(), 2, slots,
                                              heads, 1, 1, 0, out.data_ptr(), out.numel(), None)
    assert rc == wrs._lib.WRS_EINVAL
    arena.close()
