"""GPU regression tests of the runtime's edge paths: decode over a layer
without cross K/V, device zero fills for empty key sets, per-layer cross
lengths, and context scratch that is sized before graph capture (and refused
during it)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note

pytestmark = pytest.mark.gpu


@pytest.fixture()
def fresh_ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    yield c
    c.close()


def test_decode_cross_without_cross_plane_is_zero(wrs, fresh_ctx):
    # An arena created with n_audio_max = 0 has no cross planes at all; the
    # reference returns zeros for t_kv == 0 (attention.rs:93-96).
    note("decode_cross on an arena with n_audio_max = 0")
    H, beams = 4, 5
    arena = wrs.KvArena(2, 1, H, 16, 0, ctx=fresh_ctx)
    q = torch.randn((beams, H * 64), device="cuda")
    out = torch.full((beams, H * 64), float("nan"), device="cuda")
    arena.decode_cross(1, q, out)
    assert np.array_equal(host(out), np.zeros((beams, H * 64), np.float32))
    arena.close()


def test_decode_and_prefill_cross_after_invalidate_are_zero(wrs, fresh_ctx):
    note("decode_cross / prefill_cross after invalidate_cross")
    from wrs_amd import workloads as W
    H, n_audio = 2, 300
    arena = wrs.KvArena(1, 1, H, 16, n_audio, ctx=fresh_ctx)
    k = W.normal((n_audio, H * 64), 1, storage="f16")
    arena.set_cross(0, dev(k), dev(k))
    arena.invalidate_cross()
    assert arena.cross_len(0) == 0
    q = torch.randn((3, H * 64), device="cuda")
    for n in (1, 3):
        out = torch.full((n, H * 64), float("nan"), device="cuda")
        if n == 1:
            arena.decode_cross(0, q[:1], out)
        else:
            arena.prefill_cross(0, q[:n], out)
        assert np.array_equal(host(out), np.zeros((n, H * 64), np.float32)), n
    arena.close()


def test_cross_len_is_per_layer(wrs, fresh_ctx):
    # DecoderKvCache keeps cross K/V per layer (decoder.rs:136-139).
    note("cross_len per layer")
    arena = wrs.KvArena(3, 1, 1, 8, 64, ctx=fresh_ctx)
    rows = np.ones((40, 64), np.float32)
    arena.set_cross(1, rows, rows)
    assert [arena.cross_len(l) for l in range(3)] == [0, 40, 0]
    with pytest.raises(RuntimeError):
        arena.cross_len(3)
    arena.close()


def test_prefill_with_no_keys_zero_fills_strided_rows(wrs, fresh_ctx):
    # t_kv == 0 zero-fills the output (attention.rs:93-96) through a fill
    # kernel; columns outside the heads' [t_q][d_head] blocks stay untouched.
    note("prefill t_kv = 0 zero fill, strided output")
    B, H, T, dh = 2, 3, 5, 64
    row = H * dh + 16
    out = torch.full((B, T, row), 7.0, device="cuda")
    q = torch.randn((B, T, H * dh), device="cuda")
    lq = wrs.token_major(T, H * dh, dh)
    lo = wrs.Layout(T * row, dh, row)
    wrs.prefill(q, q, q, out, batch=B, n_heads=H, t_q=T, t_kv=0, d_head=dh, q_layout=lq,
                kv_layout=lq, out_layout=lo, ctx=fresh_ctx)
    got = host(out)
    assert np.array_equal(got[:, :, :H * dh], np.zeros((B, T, H * dh), np.float32))
    assert np.array_equal(got[:, :, H * dh:], np.full((B, T, 16), 7.0, np.float32))


def _decode_setup(wrs, ctx, W):
    H, n_audio, beams = 4, 1500, 5
    cross = wrs.KvArena(1, 1, H, 448, n_audio, ctx=ctx)
    k = W.normal((n_audio, H * 64), 11, storage="f16")
    v = W.normal((n_audio, H * 64), 12, storage="f16")
    cross.set_cross(0, dev(k), dev(v))
    slots = 5
    selfa = wrs.KvArena(1, slots, H, 448, 0, ctx=ctx)
    ks = W.normal((400, H * 64), 13, storage="f16")
    for s_ in range(slots):
        selfa.append(0, s_, dev(ks[:300 + 20 * s_]), dev(ks[:300 + 20 * s_]))
        selfa.advance(s_, 300 + 20 * s_ - 1)
    q = torch.from_numpy(W.normal((beams, H * 64), 14)).cuda()
    return H, beams, slots, cross, selfa, q


def test_reserved_scratch_allows_graph_capture(wrs, fresh_ctx):
    # Sized before capture, the split-K decode allocates nothing while a graph
    # records it; replays (with eager work between them) match eager calls.
    from wrs_amd import workloads as W
    note("reserve + graph capture of decode_cross / decode_self")
    ctx = fresh_ctx
    H, beams, slots, cross, selfa, q = _decode_setup(wrs, ctx, W)
    ctx.reserve(n_heads=H, decode_rows=slots, decode_keys=1500)
    out_c = torch.zeros((beams, H * 64), device="cuda")
    out_s = torch.zeros((slots, H * 64), device="cuda")
    cross.decode_cross(0, q, out_c)
    selfa.decode_self(0, list(range(slots)), q, out_s)
    ref_c, ref_s = out_c.clone(), out_s.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        cross.decode_cross(0, q, out_c)
        selfa.decode_self(0, list(range(slots)), q, out_s)
    ctx.use_torch_stream()
    for rep in range(3):
        out_c.fill_(float("nan"))
        out_s.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_c, ref_c), f"replay {rep}: cross decode differs from eager"
        assert torch.equal(out_s, ref_s), f"replay {rep}: self decode differs from eager"
        # eager work between replays
        cross.decode_cross(0, q * 0.5, out_c)
        torch.cuda.synchronize()
    cross.close()
    selfa.close()


def test_scratch_growth_during_capture_is_refused(wrs, fresh_ctx):
    from wrs_amd import workloads as W
    note("decode_cross during capture without reserved scratch -> WRS_ECAPTURE")
    ctx = fresh_ctx
    H, beams, slots, cross, selfa, q = _decode_setup(wrs, ctx, W)
    out_c = torch.zeros((beams, H * 64), device="cuda")
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="reserve"):
        with torch.cuda.graph(g):
            out_c.add_(0.0)  # the graph is not empty when the capture ends
            ctx.use_torch_stream()
            cross.decode_cross(0, q, out_c)
    ctx.use_torch_stream()
    torch.cuda.synchronize()
    # outside capture the same call sizes its scratch and runs
    cross.decode_cross(0, q, out_c)
    ref = np.zeros((beams, H * 64), np.float32)
    torch.cuda.synchronize()
    assert np.isfinite(host(out_c)).all() and maxerr(host(out_c), ref) < 10
    cross.close()
    selfa.close()


def test_split_prefill_under_graph_capture(wrs, fresh_ctx):
    # One whisper-base window (96 blocks of 128 queries, fewer than half the
    # CUs) splits each block over two workgroups through context scratch that
    # the first call outside capture allocates. Captured before that call,
    # the prefill takes the key split instead (no allocation, no error);
    # captured after it, the split blocks replay bit-identically to eager
    # calls, with eager work between the replays.
    from wrs_amd import workloads as W
    note("16-bit prefill of one whisper-base window under graph capture")
    ctx = fresh_ctx
    H, T = 8, 1500
    x = [dev(W.normal((T, H * 64), 40 + i, storage="f16"), torch.float16) for i in range(3)]
    lay = wrs.token_major(T, H * 64, 64)
    out = torch.zeros((T, H * 64), device="cuda")

    def run():
        wrs.prefill(x[0], x[1], x[2], out, batch=1, n_heads=H, t_q=T, t_kv=T, d_head=64,
                    q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)

    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0):
        ctx.use_torch_stream()
        run()
    ctx.use_torch_stream()
    out.fill_(float("nan"))
    g0.replay()
    torch.cuda.synchronize()
    before = out.clone()
    run()  # outside capture: allocates the scratch, runs the split blocks
    torch.cuda.synchronize()
    ref = out.clone()
    assert torch.isfinite(ref).all()
    assert maxerr(host(before), host(ref)) < 1e-4, "key split and split blocks disagree"
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        ctx.use_torch_stream()
        run()
    ctx.use_torch_stream()
    for rep in range(3):
        out.fill_(float("nan"))
        g1.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: split prefill differs from eager"
        run()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"eager call after replay {rep} differs"


def test_f32_workgroup_split_under_graph_capture(wrs, fresh_ctx):
    # flash_attention_2's (64, 1500) x 6 heads shape in f32: each 32-query
    # block's key tiles go to 12 workgroups folded through the same context
    # scratch. Captured before any eager call the launch keeps one workgroup
    # per block (no allocation); captured after, it replays the workgroup
    # split bit-identically to eager calls, with eager work between replays.
    note("f32 prefill (64, 1500) x 6 heads under graph capture")
    ctx = fresh_ctx
    H, TQ, TK = 6, 64, 1500
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q = torch.randn((TQ, H * 64), generator=g, device="cuda")
    k = torch.randn((TK, H * 64), generator=g, device="cuda")
    v = torch.randn((TK, H * 64), generator=g, device="cuda")
    lq, lk = wrs.token_major(TQ, H * 64, 64), wrs.token_major(TK, H * 64, 64)
    out = torch.zeros((TQ, H * 64), device="cuda")

    def run():
        wrs.prefill(q, k, v, out, batch=1, n_heads=H, t_q=TQ, t_kv=TK, d_head=64,
                    q_layout=lq, kv_layout=lk, out_layout=lq, ctx=ctx)

    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0):
        ctx.use_torch_stream()
        run()
    ctx.use_torch_stream()
    out.fill_(float("nan"))
    g0.replay()
    torch.cuda.synchronize()
    before = out.clone()
    run()  # outside capture: allocates the scratch, runs the workgroup split
    torch.cuda.synchronize()
    ref = out.clone()
    assert torch.isfinite(ref).all()
    assert maxerr(host(before), host(ref)) < 1e-5, "one and twelve workgroups per block disagree"
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        ctx.use_torch_stream()
        run()
    ctx.use_torch_stream()
    for rep in range(3):
        out.fill_(float("nan"))
        g1.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: f32 workgroup split differs from eager"
        run()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"eager call after replay {rep} differs"
