"""GPU parity of the DTW alignment-head capture
(capture_cross_attention_heads, crates/whisper/src/decoder.rs:796-828) over the
f16 cross plane of the device KV arena, against the CPU oracle run on the same
f16-rounded keys."""
from __future__ import annotations

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
