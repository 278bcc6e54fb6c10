"""GPU parity of the prefill path (encoder self-attention, prompt rows) against
the CPU oracle, through the C ABI.

Bars: 1e-5 max-abs for f32 inputs (the reference's own tiled-vs-materialized
bound, crates/tensor/tests/test_flash_attention_tiled.rs:126), 2e-3 for
f16/bf16 inputs (values widened exactly to f32 for the oracle).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, maxerr, note
from refmath import attention_f64
from test_oracle import KAT_SHAPES, _kat_inputs, _modular_inputs

pytestmark = pytest.mark.gpu

TOL16 = 2e-3
TOL32 = 1e-5


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


@pytest.fixture(params=[0, 32, -2, -3, -128, -192, -256, 128, 256],
                ids=["default", "ks32", "ws2", "ws3", "kh128", "kh192", "kh256", "wg128", "wg256"])
def schedule(request, ctx):
    """Every schedule of the 16-bit kernel on the same shapes: 4-wave
    workgroups of 256 or 128 queries, blocks of 256, 192 or 128 queries on
    8 or 12 waves whose halves take alternate 64-key tiles (key halves,
    -256 / -192 / -128), 128-query blocks split over two or three such
    workgroups and merged through memory (-2 / -3), and the key split (32
    queries, four waves over the keys); and the default, by which the grid
    size picks one."""
    ctx.set_schedule(prefill_queries=request.param)
    yield request.param
    ctx.set_schedule()


@pytest.fixture(params=[-1, 0, 1, 3, 5],
                ids=["f32default", "f32block", "f32ksplit", "f32ksplit3", "f32ksplitws"])
def f32_schedule(request, ctx):
    """The schedules of the f32 kernel on the same shapes: the key-split
    workgroups by default (32 queries, key tiles interleaved over four waves;
    three when forced to 3), 128-query blocks when forced (0); grids of fewer
    32-query blocks than half the CUs spread each block over several key-split
    workgroups (forced: 5)."""
    ctx.set_schedule(f32_split=request.param)
    yield request.param
    ctx.set_schedule()


def _oracle_fa2(orc, q, k, v, t_q, t_kv, n_heads, d_model, causal=False):
    out = np.zeros(t_q * d_model, np.float32)
    orc.flash_attention_2(np.ascontiguousarray(q.ravel()), np.ascontiguousarray(k.ravel()),
                          np.ascontiguousarray(v.ravel()), t_q, t_kv, n_heads, d_model, causal,
                          out)
    return out.reshape(t_q, d_model)


# ---- host-slice drop-in: the reference's own known-answer tests -----------

@pytest.mark.parametrize("t_q,t_kv,h,dh,causal", KAT_SHAPES)
def test_host_slice_kat(wrs, orc, ctx, t_q, t_kv, h, dh, causal, f32_schedule):
    note(f"host-slice flash_attention_2 t_q={t_q} t_kv={t_kv} h={h} dh={dh} causal={causal}")
    d_model, q, k, v = _kat_inputs(orc, t_q, t_kv, h, dh)
    out = np.full(t_q * d_model, np.nan, np.float32)
    wrs.flash_attention_2(q, k, v, t_q, t_kv, h, d_model, causal, out, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, h, d_model, causal)
    orc_out = _oracle_fa2(orc, q, k, v, t_q, t_kv, h, d_model, causal)
    assert maxerr(out.reshape(t_q, d_model), orc_out) <= TOL32
    assert maxerr(out.reshape(t_q, d_model), ref) <= TOL32


@pytest.mark.parametrize("dh,causal", [(32, False), (96, True), (128, False), (128, True),
                                       (33, False), (75, True)])
def test_host_slice_head_sizes(wrs, orc, ctx, dh, causal, f32_schedule):
    # d_head 32, 96 and 128: one, three and four 32-wide d blocks, rows of exactly
    # that many floats (the key split's float4 row loads); 33 and 75: odd widths
    # (element loads, and the workgroup split's fold one float at a time)
    t_q, t_kv, h = 70, 133, 3
    d_model = h * dh
    note(f"host-slice flash_attention_2 d_head={dh} causal={causal}")
    rng = orc.Rng(0x5EED ^ dh)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.full(t_q * d_model, np.nan, np.float32)
    wrs.flash_attention_2(q, k, v, t_q, t_kv, h, d_model, causal, out, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, h, d_model, causal)
    assert maxerr(out.reshape(t_q, d_model), ref) <= TOL32
    assert maxerr(out.reshape(t_q, d_model),
                  _oracle_fa2(orc, q, k, v, t_q, t_kv, h, d_model, causal)) <= TOL32


@pytest.mark.parametrize("causal", [False, True])
def test_host_slice_modular_inputs(wrs, orc, ctx, causal, f32_schedule):
    # crates/tensor/tests/test_flash_attention.rs:3-98 (d_head 16, bound 1e-4)
    t_q, t_kv, n_heads, d_model = 64, 128, 4, 64
    note(f"host-slice modular inputs causal={causal}")
    q, k, v = _modular_inputs(t_q, t_kv, d_model)
    out = np.zeros(t_q * d_model, np.float32)
    wrs.multi_head_attention(q, k, v, t_q, t_kv, n_heads, d_model, causal, out, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, n_heads, d_model, causal)
    assert maxerr(out.reshape(t_q, d_model), ref) <= 1e-4
    assert maxerr(out.reshape(t_q, d_model),
                  _oracle_fa2(orc, q, k, v, t_q, t_kv, n_heads, d_model, causal)) <= TOL32


def test_host_slice_causal_single_query_sees_first_key(wrs, orc, ctx, f32_schedule):
    # test_flash_attention_tiled.rs:186-205
    note("host-slice causal single query")
    d_model, t_kv = 64, 17
    rng = orc.Rng(0xFEED_FACE)
    q, k, v = rng.fill(d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.zeros(d_model, np.float32)
    wrs.flash_attention_2(q, k, v, 1, t_kv, 1, d_model, True, out, ctx=ctx)
    assert np.all(np.abs(out - v[:d_model]) <= 1e-6)


def test_host_slice_overwrites_stale_output(wrs, orc, ctx, f32_schedule):
    # test_flash_attention_tiled.rs:243-262
    note("host-slice stale NaN sentinel")
    t_q, t_kv, n_heads, d_model = 40, 100, 2, 128
    rng = orc.Rng(0xDEAD_BEEF)
    q, k, v = rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)
    out = np.full(t_q * d_model, np.nan, np.float32)
    wrs.flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model, True, out, ctx=ctx)
    assert np.all(np.isfinite(out))


def test_host_slice_edges_and_asserts(wrs, ctx):
    note("host-slice edge cases")
    d_model = 128
    k = np.ones(5 * d_model, np.float32)
    # t_q == 0: no-op (attention.rs:90-92)
    wrs.flash_attention_2(np.zeros(0, np.float32), k, k, 0, 5, 2, d_model, False,
                          np.zeros(0, np.float32), ctx=ctx)
    # t_kv == 0: zero fill (attention.rs:93-96)
    out = np.full(3 * d_model, np.nan, np.float32)
    e = np.zeros(0, np.float32)
    wrs.flash_attention_2(np.ones(3 * d_model, np.float32), e, e, 3, 0, 2, d_model, False, out,
                          ctx=ctx)
    assert np.all(out == 0.0)
    q = np.zeros(d_model, np.float32)
    with pytest.raises(AssertionError):  # n_heads == 0 (attention.rs:79)
        wrs.flash_attention_2(q, q, q, 1, 1, 0, d_model, False, q.copy(), ctx=ctx)
    with pytest.raises(AssertionError):  # d_model % n_heads (:80-83)
        wrs.flash_attention_2(q, q, q, 1, 1, 3, d_model, False, q.copy(), ctx=ctx)
    with pytest.raises(AssertionError):  # q.len() != t_q*d_model (:85)
        wrs.flash_attention_2(q, q, q, 2, 1, 2, d_model, False, q.copy(), ctx=ctx)


# ---- device-resident prefill on the benchmark-shaped workloads ------------

def _encoder_run(wrs, ctx, cfg, q, k, v, dtype, batch=None):
    b = q.shape[0] if batch is None else batch
    T, dm = cfg.t, cfg.d_model
    qd, kd, vd = dev(q, dtype), dev(k, dtype), dev(v, dtype)
    out = torch.full((b, T, dm), float("nan"), dtype=torch.float32, device="cuda")
    lay = wrs.token_major(T, dm, 64)
    wrs.prefill(qd, kd, vd, out, batch=b, n_heads=cfg.n_heads, t_q=T, t_kv=T, d_head=64,
                q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
    return host(out)


def test_tiny_encoder_f32(wrs, orc, ctx, f32_schedule):
    from wrs_amd import workloads as W
    cfg = W.TINY_ENCODER
    note(f"device prefill f32: {cfg.name}")
    q, k, v = cfg.inputs()
    out = _encoder_run(wrs, ctx, cfg, q, k, v, torch.float32)
    ref = _oracle_fa2(orc, q[0], k[0], v[0], cfg.t, cfg.t, cfg.n_heads, cfg.d_model)
    assert maxerr(out[0], ref) <= TOL32


def test_base_encoder_f16(wrs, orc, ctx, schedule):
    from wrs_amd import workloads as W
    cfg = W.BASE_ENCODER
    note(f"device prefill f16 MFMA: {cfg.name}")
    q, k, v = cfg.inputs()
    out = _encoder_run(wrs, ctx, cfg, q, k, v, torch.float16)
    for w in range(cfg.batch):
        ref = _oracle_fa2(orc, q[w], k[w], v[w], cfg.t, cfg.t, cfg.n_heads, cfg.d_model)
        assert maxerr(out[w], ref) <= TOL16, f"window {w}"


def test_large_encoder_bf16(wrs, orc, ctx, schedule):
    from wrs_amd import workloads as W
    cfg = W.LARGE_ENCODER
    note(f"device prefill bf16 MFMA: {cfg.name}")
    q, k, v = cfg.inputs()
    out = _encoder_run(wrs, ctx, cfg, q, k, v, torch.bfloat16)
    assert np.all(np.isfinite(out))
    # every window, all 20 heads, against the oracle; the worst error of each
    # window is printed (pytest -s) before the bound is checked
    worst = []
    for w in range(cfg.batch):
        ref = _oracle_fa2(orc, q[w], k[w], v[w], cfg.t, cfg.t, cfg.n_heads, cfg.d_model)
        worst.append(maxerr(out[w], ref))
        note(f"  window {w:2d}: max|gpu - oracle| = {worst[-1]:.3e}")
    assert max(worst) <= TOL16, [f"{e:.3e}" for e in worst]
    # every window: each output is a convex combination of that head's V rows
    vmin = v.min(axis=1)
    vmax = v.max(axis=1)
    assert np.all(out >= vmin[:, None, :] - 1e-3) and np.all(out <= vmax[:, None, :] + 1e-3)
    # a window computed alone equals the same window inside the batch, bitwise
    # under one schedule; by default the grid size picks the schedule, and the
    # two grids round the weights against different running maxima, each
    # within TOL16 of the oracle
    note("device prefill bf16: window 7 alone")
    alone = _encoder_run(wrs, ctx, cfg, q[7:8], k[7:8], v[7:8], torch.bfloat16, batch=1)
    if schedule == 0:
        assert maxerr(alone[0], out[7]) <= 2 * TOL16
    else:
        assert np.array_equal(alone[0], out[7])


@pytest.mark.parametrize("t", [1000, 1500])
def test_prefill_many_query_blocks(wrs, ctx, t, schedule):
    # Several rounds of workgroups (640 query blocks): every window of the
    # batch equals the same window run alone, bitwise (with the workgroup size
    # fixed: the two sizes round differently), and matches the float64
    # reference.
    from wrs_amd import workloads as W
    B, H = 40, 4
    dm = H * 64
    note(f"device prefill f16 many blocks: batch {B} heads {H} t {t}")
    q = W.normal((B, t, dm), 80, storage="f16")
    k = W.normal((B, t, dm), 81, storage="f16")
    v = W.normal((B, t, dm), 82, storage="f16")
    k[:, ::7] *= 2.0  # spread the row maxima over the key range (exact in f16)
    lay = wrs.token_major(t, dm, 64)
    qd, kd, vd = dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16)
    out = torch.full((B, t, dm), float("nan"), dtype=torch.float32, device="cuda")
    wrs.prefill(qd, kd, vd, out, batch=B, n_heads=H, t_q=t, t_kv=t, d_head=64, q_layout=lay,
                kv_layout=lay, out_layout=lay, ctx=ctx)
    got = host(out)
    assert np.all(np.isfinite(got))
    one = torch.full((1, t, dm), float("nan"), dtype=torch.float32, device="cuda")
    for b in range(B):
        wrs.prefill(qd[b:b + 1], kd[b:b + 1], vd[b:b + 1], one, batch=1, n_heads=H, t_q=t,
                    t_kv=t, d_head=64, q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
        if schedule == 0:  # the two grids may take different schedules
            assert maxerr(got[b], host(one)[0]) <= 2 * TOL16, f"window {b}"
        else:
            assert np.array_equal(got[b], host(one)[0]), f"window {b}"
    for b in (0, 17, B - 1):
        ref = attention_f64(q[b], k[b], v[b], t, t, H, dm)
        assert maxerr(got[b], ref) <= TOL16, f"window {b}"


def test_fused_qkv_row_layout(wrs, ctx):
    # q/k/v as column slices of one [B][T][3*d_model] projection output
    # (crates/whisper/src/encoder.rs:275-287) give the same bits as packed rows.
    from wrs_amd import workloads as W
    B, H, T = 2, 8, 300
    dm = H * 64
    note("device prefill f16: fused QKV row layout")
    x = W.normal((B, T, 3 * dm), 7, storage="f16")
    xd = dev(x, torch.float16)
    out_a = torch.empty((B, T, dm), dtype=torch.float32, device="cuda")
    la = wrs.token_major(T, dm, 64, row_stride=3 * dm)
    lo = wrs.token_major(T, dm, 64)
    wrs.prefill(xd[..., :dm], xd[..., dm:2 * dm], xd[..., 2 * dm:], out_a, batch=B, n_heads=H,
                t_q=T, t_kv=T, d_head=64, q_layout=la, kv_layout=la, out_layout=lo, ctx=ctx)
    qd = xd[..., :dm].contiguous()
    kd = xd[..., dm:2 * dm].contiguous()
    vd = xd[..., 2 * dm:].contiguous()
    out_b = torch.empty_like(out_a)
    wrs.prefill(qd, kd, vd, out_b, batch=B, n_heads=H, t_q=T, t_kv=T, d_head=64, q_layout=lo,
                kv_layout=lo, out_layout=lo, ctx=ctx)
    assert torch.equal(out_a, out_b)


RAGGED = [(1, 1), (1, 1500), (37, 63), (128, 64), (129, 65), (300, 257), (64, 1500),
          (1500, 100)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("t_q,t_kv", RAGGED)
def test_prefill_ragged_shapes(wrs, orc, ctx, dtype, t_q, t_kv, schedule):
    from wrs_amd import workloads as W
    H = 3
    dm = H * 64
    note(f"device prefill {dtype} ragged t_q={t_q} t_kv={t_kv}")
    q = W.normal((t_q, dm), 11, storage=dtype)
    k = W.normal((t_kv, dm), 12, storage=dtype)
    v = W.normal((t_kv, dm), 13, storage=dtype)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    out = torch.full((t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
    wrs.prefill(dev(q, tdt), dev(k, tdt), dev(v, tdt), out, batch=1, n_heads=H, t_q=t_q,
                t_kv=t_kv, d_head=64, q_layout=lq, kv_layout=lk, out_layout=lq, ctx=ctx)
    ref = _oracle_fa2(orc, q, k, v, t_q, t_kv, H, dm)
    assert maxerr(host(out), ref) <= TOL16


@pytest.mark.parametrize("t_q,t_kv,offset", [(5, 12, 7), (100, 137, 37), (128, 448, 320),
                                             (90, 33, 0), (168, 37, 0)])
def test_prefill_causal_with_offset(wrs, ctx, t_q, t_kv, offset, schedule):
    from wrs_amd import workloads as W
    H = 2
    dm = H * 64
    note(f"device prefill f16 causal t_q={t_q} t_kv={t_kv} offset={offset}")
    q = W.normal((t_q, dm), 21, storage="f16")
    k = W.normal((t_kv, dm), 22, storage="f16")
    v = W.normal((t_kv, dm), 23, storage="f16")
    out = torch.full((t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
    wrs.prefill(dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16), out,
                batch=1, n_heads=H, t_q=t_q, t_kv=t_kv, d_head=64, q_layout=lq, kv_layout=lk,
                out_layout=lq, causal=True, q_pos_offset=offset, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, H, dm, causal=True, q_offset=offset)
    assert maxerr(host(out), ref) <= TOL16


def test_prefill_d_head_80_f16_inputs(wrs, ctx, f32_schedule):
    # d_head != 64 with 16-bit inputs runs the f32-MFMA kernel on widened values.
    from wrs_amd import workloads as W
    H, dh, t_q, t_kv = 2, 80, 37, 91
    dm = H * dh
    note("device prefill f16 d_head=80")
    q = W.normal((t_q, dm), 31, storage="f16")
    k = W.normal((t_kv, dm), 32, storage="f16")
    v = W.normal((t_kv, dm), 33, storage="f16")
    out = torch.zeros((t_q, dm), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, dh), wrs.token_major(t_kv, dm, dh)
    wrs.prefill(dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16), out,
                batch=1, n_heads=H, t_q=t_q, t_kv=t_kv, d_head=dh, q_layout=lq, kv_layout=lk,
                out_layout=lq, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, H, dm)
    assert maxerr(host(out), ref) <= TOL32


# ---- tile / step boundaries, layouts and rescale paths of the 16-bit kernel ----

BOUNDARY_TKV = [31, 32, 33, 95, 96, 160, 191, 192, 193, 255, 256, 257, 320, 577]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("t_kv", BOUNDARY_TKV)
def test_prefill_tile_boundaries(wrs, ctx, dtype, t_kv, schedule):
    # 1..10 key tiles, partial last steps, and three query workgroups (t_q 600)
    from wrs_amd import workloads as W
    H, t_q = 2, 600
    dm = H * 64
    note(f"device prefill {dtype} t_q={t_q} t_kv={t_kv}")
    q = W.normal((t_q, dm), 41, storage=dtype)
    k = W.normal((t_kv, dm), 42, storage=dtype)
    v = W.normal((t_kv, dm), 43, storage=dtype)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    out = torch.full((t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
    wrs.prefill(dev(q, tdt), dev(k, tdt), dev(v, tdt), out, batch=1, n_heads=H, t_q=t_q,
                t_kv=t_kv, d_head=64, q_layout=lq, kv_layout=lk, out_layout=lq, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, H, dm)
    assert maxerr(host(out), ref) <= TOL16


@pytest.mark.parametrize("t_q,t_kv,offset", [(600, 600, 0), (513, 700, 187), (260, 1500, 1240),
                                             (300, 64, 0), (257, 257, 0)])
def test_prefill_causal_workgroups(wrs, ctx, t_q, t_kv, offset, schedule):
    # causal masks across several query workgroups, first tiles masked or not
    from wrs_amd import workloads as W
    H = 2
    dm = H * 64
    note(f"device prefill bf16 causal t_q={t_q} t_kv={t_kv} offset={offset}")
    q = W.normal((t_q, dm), 51, storage="bf16")
    k = W.normal((t_kv, dm), 52, storage="bf16")
    v = W.normal((t_kv, dm), 53, storage="bf16")
    out = torch.full((t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
    wrs.prefill(dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16), out,
                batch=1, n_heads=H, t_q=t_q, t_kv=t_kv, d_head=64, q_layout=lq, kv_layout=lk,
                out_layout=lq, causal=True, q_pos_offset=offset, ctx=ctx)
    ref = attention_f64(q, k, v, t_q, t_kv, H, dm, causal=True, q_offset=offset)
    assert maxerr(host(out), ref) <= TOL16


def test_prefill_bhsd_layout(wrs, ctx):
    # [batch][head][token][64] tensors: row stride 64, head stride T*64
    from wrs_amd import workloads as W
    B, H, T = 2, 3, 333
    note("device prefill f16 BHSD layout")
    x = [W.normal((B, H, T, 64), 60 + i, storage="f16") for i in range(3)]
    lay = wrs.Layout(H * T * 64, T * 64, 64)
    out = torch.full((B, H, T, 64), float("nan"), dtype=torch.float32, device="cuda")
    wrs.prefill(dev(x[0], torch.float16), dev(x[1], torch.float16), dev(x[2], torch.float16),
                out, batch=B, n_heads=H, t_q=T, t_kv=T, d_head=64, q_layout=lay, kv_layout=lay,
                out_layout=lay, ctx=ctx)
    got = host(out)
    for b in range(B):
        for h in range(H):
            ref = attention_f64(x[0][b, h], x[1][b, h], x[2][b, h], T, T, 1, 64)
            assert maxerr(got[b, h], ref) <= TOL16, f"batch {b} head {h}"


@pytest.mark.parametrize("profile", ["ramp", "spike"])
def test_prefill_rescale_paths(wrs, ctx, profile):
    # Scores whose row max keeps jumping along the keys (ramp), or one late key
    # far above the rest (spike, weights that overflow f16 before the
    # reference max moves): the lazy rescale must still give the exact
    # softmax up to rounding.
    from wrs_amd import workloads as W
    H, t_q, t_kv = 2, 300, 900
    dm = H * 64
    note(f"device prefill f16 rescale profile={profile}")
    q = W.normal((t_q, dm), 71, storage="f32")
    k = W.normal((t_kv, dm), 72, storage="f32")
    v = W.normal((t_kv, dm), 73, storage="f16")
    q = np.abs(q)  # positive queries: the score grows with a positive key scale
    if profile == "ramp":
        k = np.abs(k) * np.linspace(0.05, 6.0, t_kv, dtype=np.float32)[:, None]
    else:
        k = k * 0.05
        k[777] = 3.0
    q = q.astype(np.float16).astype(np.float32)
    k = k.astype(np.float16).astype(np.float32)
    out = torch.full((t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
    wrs.prefill(dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16), out,
                batch=1, n_heads=H, t_q=t_q, t_kv=t_kv, d_head=64, q_layout=lq, kv_layout=lk,
                out_layout=lq, ctx=ctx)
    got = host(out)
    assert np.all(np.isfinite(got))
    ref = attention_f64(q, k, v, t_q, t_kv, H, dm)
    assert maxerr(got, ref) <= TOL16


# ---- the reference microbenchmark's shapes ------------------------------------

def _bench_inputs(orc, t_q, t_kv, d_model):
    # crates/tensor/tests/bench_flash_attention_tiled.rs:142-146: one xorshift
    # stream, q then k then v, uniform in [-1, 1]
    rng = orc.Rng(0x5EED1234)
    return rng.fill(t_q * d_model), rng.fill(t_kv * d_model), rng.fill(t_kv * d_model)


@pytest.mark.parametrize("t_q,t_kv", [(1500, 1500), (64, 1500), (4096, 4096)])
def test_host_slice_bench_shapes(wrs, orc, ctx, t_q, t_kv):
    # every (t_q, t_kv) of the reference microbenchmark, 6 heads of 64
    # (bench_flash_attention_tiled.rs:19-25), with its inputs, through the f32
    # drop-in: the oracle's tiled and materialized results at 1e-5
    H, dm = 6, 384
    note(f"host-slice flash_attention_2 t_q={t_q} t_kv={t_kv}, 6 heads, f32")
    q, k, v = _bench_inputs(orc, t_q, t_kv, dm)
    out = np.full(t_q * dm, np.nan, np.float32)
    wrs.flash_attention_2(q, k, v, t_q, t_kv, H, dm, False, out, ctx=ctx)
    tiled = np.zeros(t_q * dm, np.float32)
    orc.flash_attention_2(q, k, v, t_q, t_kv, H, dm, False, tiled)
    mat = np.zeros(t_q * dm, np.float32)
    orc.materialized_attention(q, k, v, t_q, t_kv, H, dm, mat)
    e_t, e_m = maxerr(out, tiled), maxerr(out, mat)
    note(f"  max|gpu - tiled| = {e_t:.3e}, max|gpu - materialized| = {e_m:.3e}")
    assert e_t <= TOL32 and e_m <= TOL32


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_device_prefill_bench_shape_4096(wrs, orc, ctx, dtype):
    # the same shape on the 16-bit MFMA kernel, inputs rounded to the storage
    # type and widened exactly for the oracle
    from wrs_amd import workloads as W
    t, H, dm = 4096, 6, 384
    note(f"device prefill {dtype} t_q=t_kv=4096, 6 heads")
    q, k, v = (W._round(x.reshape(t, dm), dtype) for x in _bench_inputs(orc, t, t, dm))
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    out = torch.full((t, dm), float("nan"), dtype=torch.float32, device="cuda")
    lay = wrs.token_major(t, dm, 64)
    wrs.prefill(dev(q, tdt), dev(k, tdt), dev(v, tdt), out, batch=1, n_heads=H, t_q=t, t_kv=t,
                d_head=64, q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
    ref = _oracle_fa2(orc, q, k, v, t, t, H, dm)
    e = maxerr(host(out), ref)
    note(f"  max|gpu - oracle| = {e:.3e}")
    assert e <= TOL16


# ---- bf16 V outside the f16 range: listed blocks recomputed in f32 ---------------

def _colscaled_err(got, ref, v):
    # output column d is a convex combination of V[:, d]: its f32 rounding error
    # scales with max_k |V[k, d]|
    scale = np.maximum(1.0, np.abs(v).max(axis=0))
    return float((np.abs(got - ref) / scale).max())


def _bf16_run(wrs, ctx, q, k, v, B, H, T):
    dm = H * 64
    lay = wrs.token_major(T, dm, 64)
    out = torch.full((B, T, dm), float("nan"), dtype=torch.float32, device="cuda")
    wrs.prefill(dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16), out,
                batch=B, n_heads=H, t_q=T, t_kv=T, d_head=64, q_layout=lay, kv_layout=lay,
                out_layout=lay, ctx=ctx)
    return host(out)


def test_bf16_v_beyond_f16_range(wrs, orc, ctx, schedule):
    # The 16-bit kernel widens bf16 V to f16 in LDS; |v| >= 65536 has no f16
    # value. Those blocks come out non-finite, are listed, and are recomputed by
    # the f32 kernel from the bf16 inputs, so the result is finite and matches
    # the oracle (the reference works in f32: attention.rs:68-243). Other
    # (batch, head) pairs keep the 16-bit kernel's bits, and the list is empty
    # again afterwards: a clean call repeats its first result bitwise.
    from wrs_amd import workloads as W
    B, H, T = 2, 3, 600
    dm = H * 64
    note("device prefill bf16 with V values of magnitude 1e5 in one head")
    q = W.normal((B, T, dm), 71, storage="bf16")
    k = W.normal((B, T, dm), 72, storage="bf16")
    v = W.normal((B, T, dm), 73, storage="bf16")
    clean = _bf16_run(wrs, ctx, q, k, v, B, H, T)
    big = v.copy()
    big[1, 123, 2 * 64 + 5] = 1.0e5       # batch 1, head 2
    big[1, 400, 2 * 64 + 60] = -3.0e38    # near the bf16 maximum
    big = W._round(big, "bf16")
    got = _bf16_run(wrs, ctx, q, k, big, B, H, T)
    assert np.all(np.isfinite(got))
    for b in range(B):
        ref = _oracle_fa2(orc, q[b], k[b], big[b], T, T, H, dm)
        for h in range(H):
            sl = slice(h * 64, (h + 1) * 64)
            err = maxerr(got[b][:, sl], ref[:, sl])
            rel = _colscaled_err(got[b][:, sl], ref[:, sl], big[b, :, sl])
            note(f"  batch {b} head {h}: max|gpu - oracle| = {err:.3e}, "
                 f"over max|V column| {rel:.3e}")
            if (b, h) == (1, 2):
                assert rel <= TOL32
            else:
                assert err <= TOL16
                assert np.array_equal(got[b][:, sl], clean[b][:, sl]), (b, h)
    again = _bf16_run(wrs, ctx, q, k, v, B, H, T)
    assert np.array_equal(again, clean)


def test_bf16_v_beyond_f16_range_everywhere(wrs, orc, ctx):
    # Every block of the large-v3 encoder batch (16 windows x 20 heads) meets an
    # out-of-range V value: more listed blocks than the list holds, so every
    # block is recomputed in f32. Windows 0 and 15 against the oracle.
    from wrs_amd import workloads as W
    cfg = W.LARGE_ENCODER
    note("device prefill bf16 large-v3 batch, V = 7e4 at key 700 of every head")
    q, k, v = cfg.inputs()
    v = v.copy()
    v[:, 700, ::64] = 7.0e4
    v = W._round(v, "bf16")
    out = _encoder_run(wrs, ctx, cfg, q, k, v, torch.bfloat16)
    assert np.all(np.isfinite(out))
    for w in (0, cfg.batch - 1):
        ref = _oracle_fa2(orc, q[w], k[w], v[w], cfg.t, cfg.t, cfg.n_heads, cfg.d_model)
        rel = _colscaled_err(out[w], ref, v[w])
        note(f"  window {w}: max|gpu - oracle| over max|V column| = {rel:.3e}")
        assert rel <= TOL32


@pytest.mark.parametrize("ways", [2, 3])
def test_split_blocks_repeated_launches(wrs, ctx, ways):
    # Split blocks merge through a counter per block that the merging workgroup
    # re-arms: 200 launches in a row, alternating two inputs, each give the
    # bits of the first launch with the same input (a counter left off zero
    # would make a block merge early or never).
    from wrs_amd import workloads as W
    H, T = 6, 1500
    dm = H * 64
    note(f"split blocks over {ways} workgroups: 200 launches, two alternating inputs")
    xs = [[dev(W.normal((T, dm), 90 + 3 * i + j, storage="f16"), torch.float16)
           for j in range(3)] for i in range(2)]
    lay = wrs.token_major(T, dm, 64)
    ctx.set_schedule(prefill_queries=-ways)
    try:
        outs = [torch.empty((T, dm), dtype=torch.float32, device="cuda") for _ in range(2)]
        for i in range(2):
            wrs.prefill(*xs[i], outs[i], batch=1, n_heads=H, t_q=T, t_kv=T, d_head=64,
                        q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
        ref = [host(o).copy() for o in outs]
        for i in range(2):
            assert maxerr(ref[i], attention_f64(*(host(x) for x in xs[i]), T, T, H, dm)) <= TOL16
        bad = 0
        for n in range(200):
            i = n % 2
            outs[i].fill_(float("nan"))
            wrs.prefill(*xs[i], outs[i], batch=1, n_heads=H, t_q=T, t_kv=T, d_head=64,
                        q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
            if n % 20 == 19 or n == 0:
                bad += int(not np.array_equal(host(outs[i]), ref[i]))
        torch.cuda.synchronize()
        assert bad == 0
        for i in range(2):
            assert np.array_equal(host(outs[i]), ref[i])
    finally:
        ctx.set_schedule()


def _random_shapes(n=10, seed=0x5EED_0F):
    rng = np.random.default_rng(seed)
    shapes = []
    for _ in range(n):
        causal = bool(rng.integers(2))
        shapes.append((int(rng.integers(1, 4)), int(rng.integers(1, 6)), int(rng.integers(1, 700)),
                       int(rng.integers(1, 1300)), causal,
                       int(rng.integers(0, 300)) if causal else 0,
                       "bf16" if rng.integers(2) else "f16"))
    return shapes


@pytest.mark.parametrize("B,H,t_q,t_kv,causal,offset,dtype", _random_shapes())
def test_prefill_random_shapes(wrs, ctx, B, H, t_q, t_kv, causal, offset, dtype, schedule):
    # Seeded random batch, head, length, mask and type combinations under every
    # schedule, against the float64 reference: ragged tile counts per key part,
    # partial query blocks and masked tails in one launch.
    from wrs_amd import workloads as W
    dm = H * 64
    note(f"device prefill {dtype} B={B} H={H} t_q={t_q} t_kv={t_kv} causal={causal} "
         f"offset={offset}")
    q = W.normal((B, t_q, dm), 51, storage=dtype)
    k = W.normal((B, t_kv, dm), 52, storage=dtype)
    v = W.normal((B, t_kv, dm), 53, storage=dtype)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    out = torch.full((B, t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
    wrs.prefill(dev(q, tdt), dev(k, tdt), dev(v, tdt), out, batch=B, n_heads=H, t_q=t_q,
                t_kv=t_kv, d_head=64, q_layout=lq, kv_layout=lk, out_layout=lq,
                causal=causal, q_pos_offset=offset, ctx=ctx)
    got = host(out)
    for b in range(B):
        ref = attention_f64(q[b], k[b], v[b], t_q, t_kv, H, dm, causal=causal, q_offset=offset)
        assert maxerr(got[b], ref) <= TOL16, b


def _random_f32_shapes(n=8, seed=0xF32_5EED):
    rng = np.random.default_rng(seed)
    shapes = []
    for _ in range(n):
        causal = bool(rng.integers(2))
        shapes.append((int(rng.integers(1, 3)), int(rng.integers(1, 5)), int(rng.integers(1, 300)),
                       int(rng.integers(1, 1600)), causal,
                       int(rng.integers(0, 200)) if causal else 0,
                       int(rng.choice([64, 64, 40, 96]))))
    return shapes


@pytest.mark.parametrize("B,H,t_q,t_kv,causal,offset,dh", _random_f32_shapes())
def test_prefill_random_shapes_f32(wrs, ctx, B, H, t_q, t_kv, causal, offset, dh, f32_schedule):
    # Seeded random f32 batch, head, length, width, mask and offset combinations
    # under every f32 schedule (the workgroup split included), against the
    # float64 reference at the f32 bar.
    dm = H * dh
    note(f"device prefill f32 B={B} H={H} t_q={t_q} t_kv={t_kv} dh={dh} causal={causal} "
         f"offset={offset}")
    rng = np.random.default_rng(t_q * 7919 + t_kv)
    q = rng.standard_normal((B, t_q, dm), dtype=np.float32)
    k = rng.standard_normal((B, t_kv, dm), dtype=np.float32)
    v = rng.standard_normal((B, t_kv, dm), dtype=np.float32)
    out = torch.full((B, t_q, dm), float("nan"), dtype=torch.float32, device="cuda")
    lq, lk = wrs.token_major(t_q, dm, dh), wrs.token_major(t_kv, dm, dh)
    wrs.prefill(dev(q, torch.float32), dev(k, torch.float32), dev(v, torch.float32), out,
                batch=B, n_heads=H, t_q=t_q, t_kv=t_kv, d_head=dh, q_layout=lq, kv_layout=lk,
                out_layout=lq, causal=causal, q_pos_offset=offset, ctx=ctx)
    got = host(out)
    for b in range(B):
        ref = attention_f64(q[b], k[b], v[b], t_q, t_kv, H, dm, causal=causal, q_offset=offset)
        assert maxerr(got[b], ref) <= TOL32, b
