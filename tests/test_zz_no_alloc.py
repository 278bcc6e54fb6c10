"""The allocation-free cross decode (wrs_attn_decode_cross_noalloc) against the
allocating one (wrs_attn_decode_cross): the same kernels over the library's
fixed device scratch instead of the context's, so the outputs are identical.
Two calls in a row (the second one smaller), a capture into a graph on a
context that never reserved scratch, the size limit, two contexts calling it
at once on two streams (each holds its own slot of the fixed scratch), and
the slot count (WRS_EBUSY while every slot is held, a slot freed by
wrs_attn_destroy)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note
from refmath import attention_f64

pytestmark = pytest.mark.gpu


@pytest.fixture()
def fresh_ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    yield c
    c.close()


def _arena(wrs, ctx, W, H, n_audio, seed):
    ar = wrs.KvArena(1, 1, H, 16, n_audio, ctx=ctx)
    k = W.normal((n_audio, H * 64), seed, storage="f16")
    v = W.normal((n_audio, H * 64), seed + 1, storage="f16")
    ar.set_cross(0, dev(k), dev(v))
    return ar, k, v


def test_noalloc_matches_decode_cross_twice_second_smaller(wrs, fresh_ctx):
    from wrs_amd import workloads as W
    ctx = fresh_ctx
    for H, n_audio, beams, seed in ((20, 1500, 5, 300), (6, 700, 3, 310)):
        note(f"decode_cross_noalloc H={H} n_audio={n_audio} beams={beams}")
        ar, k, v = _arena(wrs, ctx, W, H, n_audio, seed)
        q = dev(W.normal((beams, H * 64), seed + 2))
        ref = torch.full((beams, H * 64), float("nan"), device="cuda")
        got = torch.full((beams, H * 64), float("nan"), device="cuda")
        ar.decode_cross(0, q, ref)
        ar.decode_cross_noalloc(0, q, got)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        # and both within the f16 bar of the float64 result
        assert maxerr(host(got), attention_f64(host(q), k, v, beams, n_audio, H, H * 64)) <= 2e-3
        ar.close()


def test_noalloc_under_graph_capture_without_reserve(wrs, fresh_ctx):
    from wrs_amd import workloads as W
    note("decode_cross_noalloc captured on a context without reserved scratch")
    ctx = fresh_ctx
    H, n_audio, beams = 8, 1500, 5
    ar, _, _ = _arena(wrs, ctx, W, H, n_audio, 320)
    q = dev(W.normal((beams, H * 64), 322))
    out = torch.zeros((beams, H * 64), device="cuda")
    ref = torch.zeros((beams, H * 64), device="cuda")
    ar.decode_cross_noalloc(0, q, ref)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        ar.decode_cross_noalloc(0, q, out)
    ctx.use_torch_stream()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
        ar.decode_cross_noalloc(0, q * 2.0, out)  # eager work between replays
        torch.cuda.synchronize()
    ar.close()


def test_noalloc_refuses_shapes_beyond_its_scratch(wrs, fresh_ctx):
    note("decode_cross_noalloc beyond one slot (512 KiB of partials) -> WRS_ERANGE")
    ctx = fresh_ctx
    H, n_audio, beams = 64, 3000, 8  # 8 x 64 x 24 splits x 68 floats > 131072
    ar = wrs.KvArena(1, 1, H, 16, n_audio, ctx=ctx)
    rows = torch.zeros((n_audio, H * 64), device="cuda")
    ar.set_cross(0, rows, rows)
    q = torch.zeros((beams, H * 64), device="cuda")
    out = torch.zeros((beams, H * 64), device="cuda")
    with pytest.raises(RuntimeError, match="fixed scratch"):
        ar.decode_cross_noalloc(0, q, out)
    ar.decode_cross(0, q, out)  # the allocating entry point serves it
    torch.cuda.synchronize()
    assert np.array_equal(host(out), np.zeros((beams, H * 64), np.float32))
    ar.close()


def test_noalloc_two_contexts_on_two_streams_at_once(wrs):
    """Each context holds its own slot: calls of two contexts queued on two
    streams without any synchronization between them give the allocating
    entry point's bits."""
    from wrs_amd import workloads as W
    note("decode_cross_noalloc on two contexts and two streams, interleaved")
    H, n_audio, beams = 20, 1500, 5
    ctxs, arenas, qs, refs, outs, streams = [], [], [], [], [], []
    for i in range(2):
        c = wrs.Context(0)
        st = torch.cuda.Stream()
        c.set_stream(st.cuda_stream)
        ar, _, _ = _arena(wrs, c, W, H, n_audio, 400 + 10 * i)
        q = dev(W.normal((4, beams, H * 64), 402 + 10 * i))
        ref = torch.zeros((4, beams, H * 64), device="cuda")
        for r in range(4):
            ar.decode_cross(0, q[r], ref[r])
        c.synchronize()
        ctxs.append(c), arenas.append(ar), qs.append(q), refs.append(ref), streams.append(st)
        outs.append(torch.full((4, beams, H * 64), float("nan"), device="cuda"))
    torch.cuda.synchronize()
    for rep in range(3):
        for r in range(4):
            for i in range(2):
                arenas[i].decode_cross_noalloc(0, qs[i][r], outs[i][r])
        for c in ctxs:
            c.synchronize()
        for i in range(2):
            assert torch.equal(outs[i], refs[i]), f"context {i}, pass {rep}"
            outs[i].fill_(float("nan"))
        torch.cuda.synchronize()
    for ar, c in zip(arenas, ctxs):
        ar.close()
        c.set_stream(None)
        c.close()


def test_noalloc_slots_busy_then_released(wrs):
    """Four live contexts hold the four slots of the GPU; a fifth gets
    WRS_EBUSY until one of them is destroyed."""
    from wrs_amd import workloads as W
    note("decode_cross_noalloc: five contexts, four slots")
    H, n_audio, beams = 4, 512, 2
    ctxs, arenas = [], []
    q = None
    for i in range(5):
        c = wrs.Context(0)
        c.use_torch_stream()
        ar, _, _ = _arena(wrs, c, W, H, n_audio, 500 + i)
        ctxs.append(c), arenas.append(ar)
    q = dev(W.normal((beams, H * 64), 509))
    out = torch.zeros((beams, H * 64), device="cuda")
    for i in range(4):
        arenas[i].decode_cross_noalloc(0, q, out)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="held by another context"):
        arenas[4].decode_cross_noalloc(0, q, out)
    arenas[0].close()
    ctxs[0].close()
    ref = torch.zeros((beams, H * 64), device="cuda")
    arenas[4].decode_cross(0, q, ref)
    arenas[4].decode_cross_noalloc(0, q, out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for ar, c in zip(arenas[1:], ctxs[1:]):
        ar.close()
        c.close()
