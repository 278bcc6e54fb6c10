"""f32 keys and values stored into the f16 KV arena, measured against the f32
oracle.

The reference keeps its decoder caches in f32 (DecoderKvCache,
crates/whisper/src/decoder.rs:131-145); the arena stores f16
([layer][head][ctx][64]). For K/V that are not f16-representable the arena's
result therefore differs from the reference's by the storage rounding. Every
test here splits the error into

    |gpu - ref32| <= |gpu - ref16| + |ref16 - ref32|

where ref16 is the oracle on the f16-rounded K/V (the kernel's bar, 2e-3) and
ref32 the oracle on the original f32 K/V (the reference pipeline). The second
term is the storage rounding alone, computed by the oracle on the CPU. The
stated bounds for it are at whisper-large-v3 magnitudes (activations
N(0, 0.5^2) with 13 of 1280 channels x8: |q|, |k| up to ~17, scores moved by
up to ~5e-3) and at N(0, 1). The measured values are printed (pytest -s).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note, read_f16

pytestmark = pytest.mark.gpu

TOL16 = 2e-3
# |ref16 - ref32| bounds: f16 storage rounding (2^-12 relative) of K moves a
# score by up to ~|q| |k| 2^-12 / 8 ~ 5e-3 at the outlier magnitudes; V's
# rounding adds ~1e-3.
STORE_LARGE = 1.5e-2
STORE_UNIT = 1.0e-3


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


def _large_v3_act(W, shape, stream):
    x = W.normal(shape, stream, sigma=0.5)
    x[..., W.outlier_channels(shape[-1], 13)] *= np.float32(8.0)
    return x


def _f16(x):
    return x.astype(np.float16).astype(np.float32)


def _check(name, got, ref16, ref32, store_bound):
    e16, e32, store = maxerr(got, ref16), maxerr(got, ref32), maxerr(ref16, ref32)
    note(f"  {name}: |gpu-ref16| {e16:.3e}  |gpu-ref32| {e32:.3e}  |ref16-ref32| {store:.3e}")
    assert e16 <= TOL16
    assert store <= store_bound
    assert e32 <= TOL16 + store


def _planes_equal_rounded(base, off_of_head, x32, H, n):
    # the arena holds numpy's round-to-nearest-even f16 of every f32 value
    want = _f16(x32).reshape(n, H, 64)
    for h in range(H):
        got = read_f16(base, off_of_head(h), n * 64).reshape(n, 64)
        assert np.array_equal(got, want[:, h]), f"head {h}"


def test_set_cross_f32_rows_large_v3(wrs, orc, ctx):
    # set_cross (precompute_cross_attn's stores, decoder.rs:423-447) from f32
    # device rows, then the beam-5 cross decode and the DTW capture over them
    from wrs_amd import workloads as W
    H, dm, n_audio, beams = 20, 1280, 1500, 5
    note("f32 cross K/V (large-v3 magnitudes) -> f16 arena -> decode_cross, capture")
    k = _large_v3_act(W, (n_audio, dm), 500)
    v = _large_v3_act(W, (n_audio, dm), 501)
    q = _large_v3_act(W, (beams, dm), 502)
    assert not np.array_equal(k, _f16(k))
    arena = wrs.KvArena(1, 1, H, 448, n_audio, ctx=ctx)
    arena.set_cross(0, dev(k), dev(v))
    _, _, kc, vc = arena.plane_pointers()
    _planes_equal_rounded(kc, lambda h: h * n_audio * 64, k, H, n_audio)
    _planes_equal_rounded(vc, lambda h: h * n_audio * 64, v, H, n_audio)

    out = torch.full((beams, dm), float("nan"), device="cuda")
    arena.decode_cross(0, dev(q), out)
    got = host(out)
    k16, v16 = _f16(k), _f16(v)
    for b in range(beams):
        r16 = np.zeros(dm, np.float32)
        r32 = np.zeros(dm, np.float32)
        orc.single_token_mha_d64(q[b].copy(), k16.ravel().copy(), v16.ravel().copy(), n_audio,
                                 H, dm, r16)
        orc.single_token_mha_d64(q[b].copy(), k.ravel().copy(), v.ravel().copy(), n_audio, H,
                                 dm, r32)
        _check(f"decode_cross beam {b}", got[b], r16, r32, STORE_LARGE)

    # capture_cross_attention_heads (decoder.rs:796-828): softmax rows of q.k
    n_tok, sel = 4, [(0, 3), (1, 11), (2, 19)]
    qc = _large_v3_act(W, (n_tok, dm), 503)
    cap = torch.full((n_tok * 3 * n_audio,), float("nan"), device="cuda")
    arena.capture_cross_heads(0, dev(qc), sel, 3, 0, cap)
    r16 = np.zeros(n_tok * 3 * n_audio, np.float32)
    r32 = np.zeros_like(r16)
    orc.capture_cross_attention_heads(qc.ravel().copy(), k16.ravel().copy(), n_tok, n_audio, H,
                                      dm, sel, 3, 0, r16)
    orc.capture_cross_attention_heads(qc.ravel().copy(), k.ravel().copy(), n_tok, n_audio, H,
                                      dm, sel, 3, 0, r32)
    # the capture's own bar on exact keys is 1e-5
    got = host(cap)
    e16, e32, store = maxerr(got, r16), maxerr(got, r32), maxerr(r16, r32)
    note(f"  capture: |gpu-ref16| {e16:.3e}  |gpu-ref32| {e32:.3e}  |ref16-ref32| {store:.3e}")
    assert e16 <= 1e-5 and store <= STORE_LARGE and e32 <= 1e-5 + store
    arena.close()


@pytest.mark.parametrize("magnitude", ["unit", "large_v3"])
def test_append_f32_rows_self_decode(wrs, orc, ctx, magnitude):
    # kv_append of the step's f32 K/V rows (decoder.rs:631-635) and the
    # causal self-attention over the cache (decoder.rs:835-892)
    from wrs_amd import workloads as W
    H, dm, L, slots = 12, 768, 224, 5
    note(f"f32 self K/V ({magnitude}) -> f16 arena -> decode_self ctx {L}")
    if magnitude == "unit":
        mk = lambda shape, s: W.normal(shape, s)  # noqa: E731
        bound = STORE_UNIT
    else:
        mk = lambda shape, s: _large_v3_act(W, shape, s)  # noqa: E731
        bound = STORE_LARGE
    arena = wrs.KvArena(1, slots, H, 448, 0, ctx=ctx)
    kv = [(mk((L, dm), 510 + 2 * s), mk((L, dm), 511 + 2 * s)) for s in range(slots)]
    for s, (k, v) in enumerate(kv):
        arena.append(0, s, dev(k[:L - 1]), dev(v[:L - 1]))
        arena.advance(s, L - 1)
        arena.append(0, s, dev(k[L - 1:]), dev(v[L - 1:]))
    ks, vs, _, _ = arena.plane_pointers()
    for s in (0, slots - 1):
        _planes_equal_rounded(ks, lambda h: (s * H + h) * 448 * 64, kv[s][0], H, L)
        _planes_equal_rounded(vs, lambda h: (s * H + h) * 448 * 64, kv[s][1], H, L)
    q = mk((slots, dm), 530)
    out = torch.full((slots, dm), float("nan"), device="cuda")
    arena.decode_self(0, list(range(slots)), dev(q), out)
    got = host(out)
    for s, (k, v) in enumerate(kv):
        r16 = np.zeros(dm, np.float32)
        r32 = np.zeros(dm, np.float32)
        orc.mha_with_cache(q[s].copy(), _f16(k).ravel().copy(), _f16(v).ravel().copy(), 1, L,
                           L - 1, H, dm, r16)
        orc.mha_with_cache(q[s].copy(), k.ravel().copy(), v.ravel().copy(), 1, L, L - 1, H, dm,
                           r32)
        _check(f"decode_self slot {s}", got[s], r16, r32, bound)
    arena.close()


def test_set_cross_proj_against_f32_projection(wrs, orc, ctx):
    # precompute_cross_attn (decoder.rs:423-447): K = enc Wk^T, V = enc Wv^T + b
    # in f32 on the reference side, rounded to f16 once by the arena here
    from wrs_amd import workloads as W
    H, n_audio, beams = 20, 1500, 5
    dm = 64 * H
    note("cross projection (f32 sums) -> f16 arena -> decode_cross vs f32 K/V")
    rng = np.random.default_rng(540)
    enc = W.normal((n_audio, dm), 541)
    enc[:, W.outlier_channels(dm, 13)] *= np.float32(8.0)
    wk = (rng.standard_normal((dm, dm)) / np.sqrt(dm)).astype(np.float16)
    wv = (rng.standard_normal((dm, dm)) / np.sqrt(dm)).astype(np.float16)
    bv = (0.1 * rng.standard_normal(dm)).astype(np.float32)
    arena = wrs.KvArena(1, 1, H, 448, n_audio, ctx=ctx)
    arena.set_cross_proj(dev(enc), [torch.from_numpy(wk).cuda()], [torch.from_numpy(wv).cuda()],
                         [dev(bv)])
    k32 = np.zeros(n_audio * dm, np.float32)
    v32 = np.zeros(n_audio * dm, np.float32)
    orc.f16_linear(wk, dm, dm, enc.ravel(), None, n_audio, k32)
    orc.f16_linear(wv, dm, dm, enc.ravel(), bv, n_audio, v32)
    q = _large_v3_act(W, (beams, dm), 542)
    out = torch.full((beams, dm), float("nan"), device="cuda")
    arena.decode_cross(0, dev(q), out)
    got = host(out)
    for b in range(beams):
        r16 = np.zeros(dm, np.float32)
        r32 = np.zeros(dm, np.float32)
        orc.single_token_mha_d64(q[b].copy(), _f16(k32), _f16(v32), n_audio, H, dm, r16)
        orc.single_token_mha_d64(q[b].copy(), k32.copy(), v32.copy(), n_audio, H, dm, r32)
        # ref16 rounds the oracle's f32 sums; the arena rounds its own, which can
        # sit one f16 ulp away where the two sums straddle a rounding boundary
        _check(f"decode_cross beam {b}", got[b], r16, r32, STORE_LARGE)
    arena.close()
