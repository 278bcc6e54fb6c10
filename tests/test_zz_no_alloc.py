"""The allocation-free cross decode (wrs_attn_decode_cross_noalloc) against the
allocating one (wrs_attn_decode_cross): the same kernels over the library's
fixed device scratch instead of the context's, so the outputs are identical.
Two calls in a row (the second one smaller), a capture into a graph on a
context that never reserved scratch, and the size limit."""
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
    note("decode_cross_noalloc beyond 2 MiB of partials -> WRS_ERANGE")
    ctx = fresh_ctx
    H, n_audio, beams = 64, 3000, 8  # 8 x 64 x 24 splits x 68 floats > 524288
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
