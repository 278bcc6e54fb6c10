"""GPU parity of the f32 KV arena (wrs_kv_create_dtype with WRS_F32): the
reference cache's own f32 values (DecoderKvCache, decoder.rs:131-157) and the
reference's arithmetic over them -- single_token_mha_d64 and mha_with_cache on
the exact decode kernel, flash_attention_2's prompt rows on the f32 prefill
kernel, capture_cross_attention_heads with f32 scores -- against the CPU oracle
at 1e-5, and bit for bit against the host-slice entry points that run the same
kernels on token-major copies of the same values."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note, read_f32

pytestmark = pytest.mark.gpu

TOL32 = 1e-5


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


@pytest.fixture(scope="module")
def W(wrs):
    from wrs_amd import workloads
    return workloads


def _arena(wrs, ctx, n_layers, n_slots, n_heads, max_ctx, n_audio_max):
    return wrs.KvArena(n_layers, n_slots, n_heads, max_ctx, n_audio_max, ctx=ctx,
                       dtype=wrs.WRS_F32)


def _planes(ptr, base, n_heads, plane, rows):
    """Rows [0, rows) of n_heads consecutive f32 planes as [rows][n_heads*64]."""
    got = np.stack([read_f32(ptr, base + h * plane, rows * 64).reshape(rows, 64)
                    for h in range(n_heads)], axis=1)
    return got.reshape(rows, n_heads * 64)


def test_dtype_and_bad_dtype(wrs, ctx):
    note("f32 arena dtype query")
    a16 = wrs.KvArena(1, 1, 2, 16, 8, ctx=ctx)
    a32 = _arena(wrs, ctx, 1, 1, 2, 16, 8)
    assert a16.plane_dtype() == wrs.WRS_F16 and a32.plane_dtype() == wrs.WRS_F32
    with pytest.raises(AssertionError):
        wrs.KvArena(1, 1, 2, 16, 8, ctx=ctx, dtype=wrs.WRS_BF16)
    a16.close()
    a32.close()


def test_rows_are_stored_exactly_and_moved_exactly(wrs, ctx, W):
    # append (decoder.rs:631-635), copy_slot (:223-236), ensure_slots (:207-218)
    # and slide_to_fit (:248-263) keep every f32 bit of the rows
    note("f32 arena append / copy_slot / ensure_slots / slide_to_fit")
    L, H, max_ctx, n = 2, 3, 40, 29
    dm = 64 * H
    arena = _arena(wrs, ctx, L, 2, H, max_ctx, 0)
    ks = [W.normal((n, dm), 700 + l) for l in range(L)]
    vs = [W.normal((n, dm), 710 + l) for l in range(L)]
    for l in range(L):
        arena.append(l, 0, dev(ks[l]), dev(vs[l]))
    arena.advance(0, n)
    kp, vp, _, _ = arena.plane_pointers()
    plane = max_ctx * 64
    slot_stride = H * plane

    def check(slot, n_slots, rows, first):
        torch.cuda.synchronize()
        for l in range(L):
            base = (l * n_slots + slot) * slot_stride
            assert np.array_equal(_planes(kp, base, H, plane, rows), ks[l][first:first + rows])
            assert np.array_equal(_planes(vp, base, H, plane, rows), vs[l][first:first + rows])

    check(0, 2, n, 0)
    arena.copy_slot(1, 0)
    assert arena.slot_len(1) == n
    check(1, 2, n, 0)
    arena.ensure_slots(3)
    kp, vp, _, _ = arena.plane_pointers()
    check(0, 3, n, 0)
    check(1, 3, n, 0)
    pos = arena.slide_to_fit(1, 20, max_ctx)  # drops the oldest 9 rows
    assert pos == max_ctx - 20 and arena.slot_len(1) == pos
    check(1, 3, pos, n - pos)
    check(0, 3, n, 0)  # other slots untouched
    arena.close()


@pytest.mark.parametrize("lens", [(1,), (17, 1, 224), (448, 447, 300, 64, 2)])
def test_decode_self_matches_oracle_and_host_slice(wrs, orc, ctx, W, lens):
    note(f"f32 arena decode_self lens={lens}")
    H = 6
    dm = 64 * H
    arena = _arena(wrs, ctx, 2, len(lens), H, 448, 0)
    kv = []
    for s, L in enumerate(lens):
        k, v = W.normal((L, dm), 800 + s), W.normal((L, dm), 820 + s)
        kv.append((k, v))
        if L > 1:
            arena.append(1, s, dev(k[:L - 1]), dev(v[:L - 1]))
            arena.advance(s, L - 1)
        arena.append(1, s, dev(k[L - 1:]), dev(v[L - 1:]))
    q = W.normal((len(lens), dm), 840, sigma=3.0)
    out = torch.full((len(lens), dm), float("nan"), device="cuda")
    arena.decode_self(1, list(range(len(lens))), dev(q), out)
    got = host(out)
    for s, (k, v) in enumerate(kv):
        L = lens[s]
        ref = np.zeros(dm, np.float32)
        orc.mha_with_cache(q[s].copy(), k.ravel().copy(), v.ravel().copy(), 1, L, L - 1, H, dm,
                           ref)
        assert maxerr(got[s], ref) <= TOL32, f"slot {s}"
        hs = np.full(dm, np.nan, np.float32)
        wrs.mha_with_cache(q[s].copy(), k.ravel().copy(), v.ravel().copy(), 1, L, L - 1, H, dm,
                           hs, ctx=ctx)
        assert np.array_equal(got[s], hs), f"slot {s}: differs from the host-slice path"
    arena.close()


def test_decode_self_skips_tiny_weights(wrs, ctx):
    # decoder.rs:884 / attention.rs:366: weights below 1e-7 are skipped, so a
    # value of 1e4 behind a weight of ~2e-9 does not reach the output
    note("f32 arena decode_self 1e-7 skip rule")
    arena = _arena(wrs, ctx, 1, 1, 1, 8, 0)
    k = np.zeros((3, 64), np.float32)
    k[1, :] = -2.5
    v = np.zeros((3, 64), np.float32)
    v[1, :] = 1e4
    arena.append(0, 0, dev(k[:2]), dev(v[:2]))
    arena.advance(0, 2)
    arena.append(0, 0, dev(k[2:]), dev(v[2:]))
    out = torch.full((1, 64), float("nan"), device="cuda")
    arena.decode_self(0, [0], dev(np.ones((1, 64), np.float32)), out)
    assert np.abs(host(out)).max() == 0.0
    arena.close()


@pytest.mark.parametrize("n_beams,n_audio", [(1, 1), (5, 1500), (9, 1501), (2, 3000)])
def test_decode_cross_matches_oracle_and_host_slice(wrs, orc, ctx, W, n_beams, n_audio):
    note(f"f32 arena decode_cross beams={n_beams} n_audio={n_audio}")
    H = 20  # large-v3
    dm = 64 * H
    arena = _arena(wrs, ctx, 2, 1, H, 448, 3000)
    k, v = W.normal((n_audio, dm), 900), W.normal((n_audio, dm), 901)
    arena.set_cross(1, dev(k), dev(v))
    q = W.normal((n_beams, dm), 902, sigma=3.0)
    out = torch.full((n_beams, dm), float("nan"), device="cuda")
    arena.decode_cross(1, dev(q), out)
    got = host(out)
    for b in range(n_beams):
        ref = np.zeros(dm, np.float32)
        orc.single_token_mha_d64(q[b].copy(), k.ravel().copy(), v.ravel().copy(), n_audio, H, dm,
                                 ref)
        assert maxerr(got[b], ref) <= TOL32, f"beam {b}"
        hs = np.full(dm, np.nan, np.float32)
        wrs.single_token_mha_d64(q[b].copy(), k.ravel().copy(), v.ravel().copy(), n_audio, H,
                                 dm, hs, ctx=ctx)
        assert np.array_equal(got[b], hs), f"beam {b}: differs from the host-slice path"
    # a layer without cross K/V gives zero rows (attention.rs:93-96)
    out.fill_(float("nan"))
    arena.decode_cross(0, dev(q), out)
    assert np.array_equal(host(out), np.zeros((n_beams, dm), np.float32))
    arena.close()


@pytest.mark.parametrize("n_tokens,t_past", [(4, 0), (5, 7), (16, 100), (2, 446), (64, 30)])
def test_prefill_self_matches_oracle_and_host_slice(wrs, orc, ctx, W, n_tokens, t_past):
    note(f"f32 arena prefill_self n={n_tokens} t_past={t_past}")
    H = 4
    dm = 64 * H
    total = t_past + n_tokens
    arena = _arena(wrs, ctx, 1, 2, H, 448, 0)
    k, v = W.normal((total, dm), 1000), W.normal((total, dm), 1001)
    if t_past:
        arena.append(0, 1, dev(k[:t_past]), dev(v[:t_past]))
        arena.advance(1, t_past)
    arena.append(0, 1, dev(k[t_past:]), dev(v[t_past:]))
    q = W.normal((n_tokens, dm), 1002, sigma=3.0)
    out = torch.full((n_tokens, dm), float("nan"), device="cuda")
    arena.prefill_self(0, 1, dev(q), out)
    got = host(out).ravel()
    ref = np.zeros(n_tokens * dm, np.float32)
    orc.mha_with_cache(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n_tokens, total,
                       t_past, H, dm, ref)
    assert maxerr(got, ref) <= TOL32
    hs = np.full(n_tokens * dm, np.nan, np.float32)
    wrs.mha_with_cache(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n_tokens, total,
                       t_past, H, dm, hs, ctx=ctx)
    assert np.array_equal(got, hs), "differs from the host-slice path"
    arena.close()


@pytest.mark.parametrize("n_tokens,n_audio", [(1, 1500), (3, 1500), (33, 1500), (7, 37)])
def test_prefill_cross_matches_oracle(wrs, orc, ctx, W, n_tokens, n_audio):
    note(f"f32 arena prefill_cross n={n_tokens} n_audio={n_audio}")
    H = 4
    dm = 64 * H
    arena = _arena(wrs, ctx, 1, 1, H, 448, 1504)
    k, v = W.normal((n_audio, dm), 1100), W.normal((n_audio, dm), 1101)
    arena.set_cross(0, dev(k), dev(v))
    q = W.normal((n_tokens, dm), 1102, sigma=3.0)
    out = torch.full((n_tokens, dm), float("nan"), device="cuda")
    arena.prefill_cross(0, dev(q), out)
    got = host(out).ravel()
    ref = np.zeros(n_tokens * dm, np.float32)
    orc.flash_attention_2(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n_tokens,
                          n_audio, H, dm, False, ref)
    assert maxerr(got, ref) <= TOL32
    hs = np.full(n_tokens * dm, np.nan, np.float32)
    wrs.flash_attention_2(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n_tokens,
                          n_audio, H, dm, False, hs, ctx=ctx)
    assert maxerr(got, hs) <= 1e-6, "far from the host-slice path"
    arena.close()


@pytest.mark.parametrize("n_tokens,n_audio", [(1, 1), (5, 37), (9, 1500), (3, 3000)])
def test_capture_matches_oracle(wrs, orc, ctx, W, n_tokens, n_audio):
    note(f"f32 arena capture n_tokens={n_tokens} n_audio={n_audio}")
    H, n_layers = 4, 2
    dm = 64 * H
    arena = _arena(wrs, ctx, n_layers, 1, H, 448, 3000)
    ks = [W.normal((n_audio, dm), 1200 + l) for l in range(n_layers)]
    for l in range(n_layers):
        arena.set_cross(l, dev(ks[l]), dev(W.normal((n_audio, dm), 1210 + l)))
    heads = [(1, 3), (0, 2), (1, 0), (1, 3)]  # (layer, head); the same head twice
    n_sel, row_off = len(heads), 2
    q = W.normal((n_tokens, dm), 1220, sigma=2.0)
    size = (row_off + n_tokens) * n_sel * n_audio
    out = torch.full((size,), float("nan"), device="cuda")
    ref = np.full(size, np.nan, np.float32)
    for layer in range(n_layers):
        sel = [(slot, h) for slot, (l, h) in enumerate(heads) if l == layer]
        arena.capture_cross_heads(layer, dev(q), sel, n_sel, row_off, out)
        orc.capture_cross_attention_heads(q.ravel().copy(), ks[layer].ravel().copy(), n_tokens,
                                          n_audio, H, dm, sel, n_sel, row_off, ref)
    got = host(out)
    head_rows = row_off * n_sel * n_audio
    assert np.isnan(got[:head_rows]).all()  # rows before row_offset untouched
    assert maxerr(got[head_rows:], ref[head_rows:]) <= TOL32
    arena.close()


def test_cross_projection_into_f32_arena(wrs, orc, ctx, W):
    # precompute_cross_attn (decoder.rs:423-447) into f32 planes: no f16 rounding
    # of K/V; each value within the f32 accumulation bound of the oracle's
    note("cross projection into f32 arena")
    H, n_audio = 4, 1500
    dm = 64 * H
    rng = np.random.default_rng(1300)
    enc = rng.standard_normal((n_audio, dm)).astype(np.float32)
    wk = (rng.standard_normal((dm, dm)) / np.sqrt(dm)).astype(np.float16)
    wv = (rng.standard_normal((dm, dm)) / np.sqrt(dm)).astype(np.float16)
    bv = (0.1 * rng.standard_normal(dm)).astype(np.float32)
    arena = _arena(wrs, ctx, 1, 1, H, 448, n_audio)
    arena.set_cross_proj(dev(enc), [torch.from_numpy(wk).cuda()], [torch.from_numpy(wv).cuda()],
                         [dev(bv)])
    torch.cuda.synchronize()
    _, _, kc, vc = arena.plane_pointers()
    planes = {}
    for name, base, w, b in (("k", kc, wk, None), ("v", vc, wv, bv)):
        ref = np.zeros(n_audio * dm, np.float32)
        orc.f16_linear(w, dm, dm, enc.ravel(), b, n_audio, ref)
        got = _planes(base, 0, H, n_audio * 64, n_audio)
        # both sides within n 2^-23 sum |w x| of the exact product (x split
        # into two f16 parts on the GPU: products to 2^-22)
        bound = dm * 2.0 ** -23 * (np.abs(enc.astype(np.float64)) @
                                   np.abs(w.astype(np.float64)).T)
        if b is not None:
            bound = bound + 2.0 ** -22 * np.abs(b)
        assert (np.abs(got - ref.reshape(n_audio, dm)) <= 2 * bound + 2.0 ** -24).all(), name
        planes[name] = got
    q = W.normal((5, dm), 1301, sigma=3.0)
    out = torch.full((5, dm), float("nan"), device="cuda")
    arena.decode_cross(0, dev(q), out)
    got = host(out)
    for b in range(5):
        ref = np.zeros(dm, np.float32)
        orc.single_token_mha_d64(q[b].copy(), planes["k"].ravel().copy(),
                                 planes["v"].ravel().copy(), n_audio, H, dm, ref)
        assert maxerr(got[b], ref) <= TOL32, f"beam {b}"
    arena.close()


def test_f16_only_entry_points_refuse_f32_arenas(wrs, ctx, W):
    note("f32 arena: noalloc / lse entry points refuse")
    H = 2
    dm = 64 * H
    arena = _arena(wrs, ctx, 1, 1, H, 16, 64)
    arena.set_cross(0, dev(W.normal((64, dm), 1400)), dev(W.normal((64, dm), 1401)))
    q = dev(W.normal((2, dm), 1402))
    out = torch.zeros((2, dm), device="cuda")
    with pytest.raises(RuntimeError, match="unsupported"):
        arena.decode_cross_noalloc(0, q, out)
    lse = torch.zeros(2 * H * 2, device="cuda")
    with pytest.raises(RuntimeError, match="unsupported"):
        arena.prefill_cross(0, q, out, lse=lse)
    cap = torch.zeros(2 * 64, device="cuda")
    with pytest.raises(RuntimeError, match="unsupported"):
        arena.capture_cross_heads(0, q, [(0, 1)], 1, 0, cap, lse=lse)
    arena.close()
