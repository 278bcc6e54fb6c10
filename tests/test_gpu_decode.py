"""GPU parity of the decode path (single-query self- and cross-attention over
the device KV arena) and of the arena operations, against the CPU oracle and
the reference's own arena unit tests."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note, read_f16
from refmath import attention_f64

pytestmark = pytest.mark.gpu

TOL16 = 2e-3
TOL32 = 1e-5


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


# ---- host-slice drop-ins ----------------------------------------------------

@pytest.mark.parametrize("t_kv", [1, 17, 224, 1500, 1501])
def test_host_slice_single_token(wrs, orc, ctx, t_kv):
    note(f"host-slice single_token_mha_d64 t_kv={t_kv}")
    n_heads, d_model = 5, 320
    rng = orc.Rng(0xC0FFEE ^ t_kv)
    q, k, v = rng.fill(d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.full(d_model, np.nan, np.float32)
    wrs.single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, out, ctx=ctx)
    ref = np.zeros(d_model, np.float32)
    orc.single_token_mha_d64(q, k, v, t_kv, n_heads, d_model, ref)
    assert maxerr(out, ref) <= TOL32
    # the same call through flash_attention_2's t_q == 1 dispatch (attention.rs:102-105)
    out2 = np.full(d_model, np.nan, np.float32)
    wrs.flash_attention_2(q, k, v, 1, t_kv, n_heads, d_model, False, out2, ctx=ctx)
    assert np.array_equal(out, out2)


def test_host_slice_single_token_skips_tiny_weights(wrs, ctx):
    # attention.rs:366: a weight of ~2e-9 on a value of 1e4 must not reach the output.
    note("host-slice single token 1e-7 skip rule")
    d_model, t_kv = 64, 3
    q = np.full(d_model, 1.0, np.float32)
    k = np.zeros((t_kv, d_model), np.float32)
    k[1, :] = -2.5
    v = np.zeros((t_kv, d_model), np.float32)
    v[1, :] = 1e4
    out = np.zeros(d_model, np.float32)
    wrs.single_token_mha_d64(q, k.ravel(), v.ravel(), t_kv, 1, d_model, out, ctx=ctx)
    skipped = attention_f64(q, k, v, 1, t_kv, 1, d_model, skip_below=1e-7)
    assert maxerr(out, skipped.ravel()) <= 1e-7


@pytest.mark.parametrize("n_tokens,t_past,d_head", [(1, 0, 64), (1, 223, 64), (5, 7, 64),
                                                      (4, 30, 80), (1, 9, 80), (16, 100, 64)])
def test_host_slice_mha_with_cache(wrs, orc, ctx, n_tokens, t_past, d_head):
    note(f"host-slice mha_with_cache n={n_tokens} t_past={t_past} dh={d_head}")
    n_heads = 3
    d_model = n_heads * d_head
    total = t_past + n_tokens
    rng = orc.Rng(0xABCD ^ total)
    q, k, v = rng.fill(n_tokens * d_model), rng.fill(total * d_model), rng.fill(total * d_model)
    out = np.full(n_tokens * d_model, np.nan, np.float32)
    wrs.mha_with_cache(q, k, v, n_tokens, total, t_past, n_heads, d_model, out, ctx=ctx)
    ref = np.zeros(n_tokens * d_model, np.float32)
    orc.mha_with_cache(q, k, v, n_tokens, total, t_past, n_heads, d_model, ref)
    assert maxerr(out, ref) <= TOL32


def test_host_slice_mha_with_cache_asserts(wrs, ctx):
    note("host-slice mha_with_cache asserts")
    z = np.zeros(64 * 4, np.float32)
    with pytest.raises(AssertionError):  # t_past + n > total
        wrs.mha_with_cache(z[:128], z, z, 2, 4, 3, 1, 64, z[:128].copy(), ctx=ctx)
    with pytest.raises(AssertionError):  # q.len() != n*d_model (decoder.rs:847)
        wrs.mha_with_cache(z[:64], z, z, 2, 4, 2, 1, 64, z[:128].copy(), ctx=ctx)


# ---- device arena: self-attention decode (small, beam 5) ---------------------

def _fill_slot(arena, layer, slot, k, v, n_hist):
    """History rows [0, n_hist) appended and advanced; row n_hist appended only
    (the current step's row, decoder.rs:631-635 before :765-767)."""
    arena.set_len(slot, 0) if arena.slot_len(slot) else None
    if n_hist:
        arena.append(layer, slot, dev(k[:n_hist]), dev(v[:n_hist]))
        arena.advance(slot, n_hist)
    arena.append(layer, slot, dev(k[n_hist:n_hist + 1]), dev(v[n_hist:n_hist + 1]))


@pytest.mark.parametrize("L", [32, 64, 128, 224, 256, 384, 448])
def test_self_decode_sweep(wrs, orc, ctx, L):
    from wrs_amd import workloads as W
    cfg = W.SelfDecode("small self decode", 5, 12, L)
    note(f"device decode_self beam 5 x 12 heads, ctx {L}")
    arena = wrs.KvArena(1, cfg.beams, cfg.n_heads, 448, 0, ctx=ctx)
    kvs = [cfg.kv(s) for s in range(cfg.beams)]
    for s in range(cfg.beams):
        _fill_slot(arena, 0, s, kvs[s][0], kvs[s][1], L - 1)
    q = cfg.q()
    out = torch.full((cfg.beams, cfg.d_model), float("nan"), device="cuda")
    arena.decode_self(0, list(range(cfg.beams)), dev(q), out)
    got = host(out)
    for s in range(cfg.beams):
        ref = np.zeros(cfg.d_model, np.float32)
        k, v = kvs[s]
        orc.mha_with_cache(np.ascontiguousarray(q[s]), np.ascontiguousarray(k.ravel()),
                           np.ascontiguousarray(v.ravel()), 1, L, L - 1, cfg.n_heads,
                           cfg.d_model, ref)
        assert maxerr(got[s], ref) <= TOL16, f"slot {s}"
    arena.close()


def test_self_decode_ragged_in_one_chunk(wrs, ctx):
    # Longest slot 256: every (slot, head) runs one 256-key workgroup whose
    # second tiles lie past the shorter slots' lengths, or partly inside them.
    from wrs_amd import workloads as W
    note("device decode_self ragged lengths 1..256 (256-key workgroups)")
    H, dm = 3, 192
    lens = [1, 100, 128, 129, 143, 200, 255, 256]
    arena = wrs.KvArena(1, len(lens), H, 448, 0, ctx=ctx)
    data = []
    for s, L in enumerate(lens):
        k = W.normal((L, dm), 150 + s, storage="f16")
        v = W.normal((L, dm), 170 + s, storage="f16")
        data.append((k, v))
        _fill_slot(arena, 0, s, k, v, L - 1)
    q = W.normal((len(lens), dm), 190)
    out = torch.full((len(lens), dm), float("nan"), device="cuda")
    arena.decode_self(0, list(range(len(lens))), dev(q), out)
    got = host(out)
    for s, L in enumerate(lens):
        k, v = data[s]
        ref = attention_f64(q[s], k, v, 1, L, H, dm)
        assert maxerr(got[s], ref.ravel()) <= TOL16, f"slot {s} L={L}"
    arena.close()


def test_self_decode_slot_order_and_subset(wrs, orc, ctx):
    # rows map to arbitrary slots; each slot has its own length
    from wrs_amd import workloads as W
    note("device decode_self permuted slots, ragged lengths")
    H, dm = 4, 256
    arena = wrs.KvArena(2, 6, H, 448, 0, ctx=ctx)
    lens = {5: 300, 2: 17, 0: 65}
    data = {}
    for s, L in lens.items():
        k = W.normal((L, dm), 50 + s, storage="f16")
        v = W.normal((L, dm), 60 + s, storage="f16")
        data[s] = (k, v)
        _fill_slot(arena, 1, s, k, v, L - 1)
    slots = [5, 2, 0]
    q = W.normal((3, dm), 70)
    out = torch.zeros((3, dm), device="cuda")
    arena.decode_self(1, slots, dev(q), out)
    got = host(out)
    for i, s in enumerate(slots):
        k, v = data[s]
        L = lens[s]
        ref = attention_f64(q[i], k, v, 1, L, H, dm)
        assert maxerr(got[i], ref.ravel()) <= TOL16


# ---- device arena: cross-attention decode (large-v3, beam 5) -----------------

def test_cross_decode_large_v3(wrs, orc, ctx):
    from wrs_amd import workloads as W
    cfg = W.LARGE_CROSS_DECODE
    note(f"device decode_cross: {cfg.name}, {cfg.n_layers} layers resident")
    arena = wrs.KvArena(cfg.n_layers, 1, cfg.n_heads, 448, cfg.n_audio, ctx=ctx)
    for layer in range(cfg.n_layers):
        k, v = cfg.kv(layer)
        arena.set_cross(layer, dev(k), dev(v))
    assert arena.cross_len() == cfg.n_audio
    for layer in (0, 17, cfg.n_layers - 1):
        q = cfg.q(layer)
        out = torch.full((cfg.beams, cfg.d_model), float("nan"), device="cuda")
        arena.decode_cross(layer, dev(q), out)
        got = host(out)
        k, v = cfg.kv(layer)
        for b in range(cfg.beams):
            ref = np.zeros(cfg.d_model, np.float32)
            orc.single_token_mha_d64(np.ascontiguousarray(q[b]), np.ascontiguousarray(k.ravel()),
                                     np.ascontiguousarray(v.ravel()), cfg.n_audio, cfg.n_heads,
                                     cfg.d_model, ref)
            assert maxerr(got[b], ref) <= TOL16, f"layer {layer} beam {b}"
        # the beams batched in one launch equal one launch per beam, bitwise
        for b in (0, 4):
            one = torch.zeros((1, cfg.d_model), device="cuda")
            arena.decode_cross(layer, dev(q[b:b + 1]), one)
            assert np.array_equal(host(one)[0], got[b])
    arena.close()


@pytest.mark.parametrize("beams", [1, 3, 8, 11])
def test_cross_decode_beam_counts(wrs, ctx, beams):
    from wrs_amd import workloads as W
    H, dm, n_audio = 6, 384, 700
    note(f"device decode_cross beams={beams}")
    arena = wrs.KvArena(1, 1, H, 448, 1500, ctx=ctx)
    k = W.normal((n_audio, dm), 80, storage="f16")
    v = W.normal((n_audio, dm), 81, storage="f16")
    arena.set_cross(0, k, v)  # host source path
    q = W.normal((beams, dm), 82)
    out = torch.zeros((beams, dm), device="cuda")
    arena.decode_cross(0, dev(q), out)
    got = host(out)
    ref = attention_f64(q, k, v, beams, n_audio, H, dm)
    assert maxerr(got, ref) <= TOL16
    arena.close()


@pytest.mark.parametrize("n_audio", [129, 200, 256, 257, 1536, 1537, 2900])
def test_cross_decode_split_counts(wrs, ctx, n_audio):
    # 129..256 keys: one 256-key workgroup per (beam group, head), two tiles per
    # wave, no merge. Longer planes split into 128 keys: 3, 12 (largest one-round
    # merge), 13 and 23 splits (batched merge).
    from wrs_amd import workloads as W
    H, dm, beams = 4, 256, 5
    note(f"device decode_cross n_audio={n_audio}")
    arena = wrs.KvArena(1, 1, H, 448, 3000, ctx=ctx)
    k = W.normal((n_audio, dm), 90, storage="f16")
    v = W.normal((n_audio, dm), 91, storage="f16")
    arena.set_cross(0, k, v)
    q = W.normal((beams, dm), 92)
    out = torch.full((beams, dm), float("nan"), device="cuda")
    for _ in range(2):  # the second launch reuses the re-armed counters
        arena.decode_cross(0, dev(q), out)
        got = host(out)
        ref = attention_f64(q, k, v, beams, n_audio, H, dm)
        assert maxerr(got, ref) <= TOL16
    arena.close()


# ---- prompt rows over the arena ------------------------------------------------

def test_prefill_self_prompt_rows(wrs, orc, ctx):
    # decoder.rs:857-891: n_tokens > 1 rows at offset t_past over the slot's cache
    from wrs_amd import workloads as W
    H, dm, t_past, n = 6, 384, 40, 9
    note("device prefill_self prompt rows")
    arena = wrs.KvArena(1, 2, H, 448, 0, ctx=ctx)
    k = W.normal((t_past + n, dm), 90, storage="f16")
    v = W.normal((t_past + n, dm), 91, storage="f16")
    arena.append(0, 1, dev(k[:t_past]), dev(v[:t_past]))
    arena.advance(1, t_past)
    arena.append(0, 1, dev(k[t_past:]), dev(v[t_past:]))
    q = W.normal((n, dm), 92)
    out = torch.full((n, dm), float("nan"), device="cuda")
    arena.prefill_self(0, 1, dev(q), out)
    ref = np.zeros(n * dm, np.float32)
    orc.mha_with_cache(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n, t_past + n,
                       t_past, H, dm, ref)
    assert maxerr(host(out), ref.reshape(n, dm)) <= TOL16
    arena.close()


def test_prefill_cross_prompt_rows(wrs, orc, ctx):
    from wrs_amd import workloads as W
    H, dm, n_audio, n = 6, 384, 1500, 7
    note("device prefill_cross prompt rows")
    arena = wrs.KvArena(1, 1, H, 448, n_audio, ctx=ctx)
    k = W.normal((n_audio, dm), 93, storage="f16")
    v = W.normal((n_audio, dm), 94, storage="f16")
    arena.set_cross(0, dev(k), dev(v))
    q = W.normal((n, dm), 95)
    out = torch.full((n, dm), float("nan"), device="cuda")
    arena.prefill_cross(0, dev(q), out)
    ref = np.zeros(n * dm, np.float32)
    orc.flash_attention_2(q.ravel().copy(), k.ravel().copy(), v.ravel().copy(), n, n_audio, H,
                          dm, False, ref)
    assert maxerr(host(out), ref.reshape(n, dm)) <= TOL16
    arena.close()


# ---- arena operations (decoder.rs:131-264 and its unit tests :894-925) --------

def _plane_rows(arena, layer, slot, head, n, which="k"):
    ks, vs, _, _ = arena.plane_pointers()
    base = ks if which == "k" else vs
    off = ((layer * arena.n_slots + slot) * arena.n_heads + head) * arena.max_ctx * 64
    return read_f16(base, off, n * 64).reshape(n, 64)


def test_append_converts_rows_to_head_planes(wrs, ctx):
    from wrs_amd import workloads as W
    note("arena append layout")
    H, dm = 3, 192
    arena = wrs.KvArena(2, 3, H, 16, 0, ctx=ctx)
    k = W.normal((5, dm), 1, storage="f16")
    v = W.normal((5, dm), 2, storage="f16")
    arena.append(1, 2, dev(k), dev(v))
    torch.cuda.synchronize()
    for h in range(H):
        assert np.array_equal(_plane_rows(arena, 1, 2, h, 5, "k"), k[:, h * 64:(h + 1) * 64])
        assert np.array_equal(_plane_rows(arena, 1, 2, h, 5, "v"), v[:, h * 64:(h + 1) * 64])
    arena.close()


def test_slide_to_fit_drops_oldest_rows(wrs, ctx):
    # decoder.rs:900-915, with rows of 64 per head instead of d_model 2:
    # 4 cached + 2 new against a 4-token context drop the two oldest.
    note("arena slide_to_fit")
    H, dm = 2, 128
    arena = wrs.KvArena(2, 1, H, 8, 0, ctx=ctx)
    rows = np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], dm, axis=1)
    for layer in range(2):
        arena.append(layer, 0, dev(rows), dev(rows + 10))
    arena.advance(0, 4)
    pos = arena.slide_to_fit(0, 2, 4)
    assert pos == 2 and arena.slot_len(0) == 2
    torch.cuda.synchronize()
    for layer in range(2):
        for h in range(H):
            got = _plane_rows(arena, layer, 0, h, 2, "k")
            assert np.array_equal(got, np.repeat(np.array([[3.0], [4.0]], np.float32), 64, 1))
            got = _plane_rows(arena, layer, 0, h, 2, "v")
            assert np.array_equal(got, np.repeat(np.array([[13.0], [14.0]], np.float32), 64, 1))
    arena.close()


def test_slide_to_fit_is_a_noop_when_room_exists(wrs, ctx):
    # decoder.rs:917-925
    note("arena slide_to_fit no-op")
    arena = wrs.KvArena(1, 1, 1, 8, 0, ctx=ctx)
    rows = np.ones((3, 64), np.float32)
    arena.append(0, 0, dev(rows), dev(rows))
    arena.advance(0, 3)
    assert arena.slide_to_fit(0, 1, 8) == 3
    assert arena.slot_len(0) == 3
    arena.close()


def test_slide_long_history(wrs, ctx):
    # a drop smaller than the 32-row move block and a long kept range
    from wrs_amd import workloads as W
    note("arena slide 448 -> keep 441")
    H, dm = 2, 128
    arena = wrs.KvArena(1, 1, H, 448, 0, ctx=ctx)
    k = W.normal((448, dm), 5, storage="f16")
    arena.append(0, 0, dev(k), dev(k))
    arena.advance(0, 448)
    assert arena.slide_to_fit(0, 7, 448) == 441
    torch.cuda.synchronize()
    for h in range(H):
        assert np.array_equal(_plane_rows(arena, 0, 0, h, 441), k[7:, h * 64:(h + 1) * 64])
    arena.close()


def test_copy_slot_and_rewind(wrs, ctx):
    from wrs_amd import workloads as W
    note("arena copy_slot / set_len / clear_slot / ensure_slots")
    H, dm = 2, 128
    arena = wrs.KvArena(3, 2, H, 64, 0, ctx=ctx)
    k = W.normal((20, dm), 6, storage="f16")
    for layer in range(3):
        arena.append(layer, 0, dev(k), dev(k * 2))
    arena.advance(0, 20)
    arena.copy_slot(1, 0)  # beam fork (beam.rs:455)
    assert arena.slot_len(1) == 20
    torch.cuda.synchronize()
    for layer in range(3):
        assert np.array_equal(_plane_rows(arena, layer, 1, 1, 20), k[:, 64:])
        assert np.array_equal(_plane_rows(arena, layer, 1, 0, 20, "v"), (k * 2)[:, :64])
    arena.set_len(1, 5)  # n_past rewind (ffi lib.rs:2352)
    assert arena.slot_len(1) == 5
    with pytest.raises(AssertionError):
        arena.set_len(1, 6)  # rows past the stored history do not exist
    arena.ensure_slots(5)  # grows, keeps contents (decoder.rs:207-218)
    assert arena.slot_len(0) == 20 and arena.slot_len(4) == 0
    torch.cuda.synchronize()
    for layer in range(3):
        assert np.array_equal(_plane_rows(arena, layer, 0, 1, 20), k[:, 64:])
    arena.clear_slot(0)
    assert arena.slot_len(0) == 0 and arena.slot_len(1) == 5
    arena.clear()
    assert arena.slot_len(1) == 0
    with pytest.raises(RuntimeError):
        arena.copy_slot(7, 0)  # slot out of range
    arena.close()


def test_invalidate_cross(wrs, ctx):
    note("arena invalidate_cross")
    arena = wrs.KvArena(1, 1, 1, 8, 32, ctx=ctx)
    rows = np.ones((32, 64), np.float32)
    arena.set_cross(0, rows, rows)
    assert arena.cross_len() == 32
    arena.invalidate_cross()
    assert arena.cross_len() == 0
    arena.close()
