"""GPU parity of the f16-weight projections (LinearWeight::linear with F16
weights: crates/tensor/src/ops/quant.rs:415-473) through the C ABI, against the
CPU oracle's f16_linear on the same inputs: the plain projection, the fused
QKV projection feeding the encoder attention in place (encoder.rs:275-299), and
the cross K/V precompute into the arena (decoder.rs:423-447)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, note, read_f16
from refmath import attention_f64

pytestmark = pytest.mark.gpu

TOL16 = 2e-3


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


def _weights(rows, cols, seed, scale=None):
    rng = np.random.default_rng(seed)
    s = (1.0 / np.sqrt(cols)) if scale is None else scale
    return (s * rng.standard_normal((rows, cols))).astype(np.float16)


def _gamma_bound(x, w):
    """n * 2^-23 * sum_k |w_rk x_tk|: the f32 accumulation bound both sides obey."""
    return x.shape[1] * 2.0 ** -23 * (np.abs(x.astype(np.float64)) @
                                      np.abs(w.astype(np.float64)).T)


def _rounded_tol(x, w, r, out_dt):
    """|round(a) - round(b)| <= |a - b| + spacing: two f32 sums within the
    accumulation bound each, rounded to the output type r is in."""
    rel = 2.0 ** -10 if out_dt == "f16" else 2.0 ** -7
    return 2 * _gamma_bound(x, w) + np.abs(r) * rel + 2.0 ** -24


def _exact(x, w, b):
    y = x.astype(np.float64) @ w.astype(np.float64).T
    return y if b is None else y + b


@pytest.mark.parametrize("n_tokens,n_in,n_out,use_bias", [
    (1, 64, 4, False), (5, 384, 68, True), (127, 384, 1152, True), (129, 512, 512, False),
    (300, 1280, 1284, True), (1500, 1280, 3840, True)])
def test_linear_f32_matches_oracle(wrs, orc, ctx, n_tokens, n_in, n_out, use_bias):
    note(f"linear f32 T={n_tokens} K={n_in} N={n_out} bias={use_bias}")
    rng = np.random.default_rng(n_tokens * 7 + n_out)
    x = (3.0 * rng.standard_normal((n_tokens, n_in))).astype(np.float32)
    w = _weights(n_out, n_in, n_in + n_out)
    b = rng.standard_normal(n_out).astype(np.float32) if use_bias else None
    out = torch.full((n_tokens, n_out), float("nan"), device="cuda")
    wrs.linear(dev(x), torch.from_numpy(w).cuda(), None if b is None else dev(b), out, ctx=ctx)
    got = host(out).astype(np.float64)
    ref = np.zeros(n_tokens * n_out, np.float32)
    orc.f16_linear(w, n_out, n_in, x.ravel(), b, n_tokens, ref)
    ref = ref.reshape(n_tokens, n_out).astype(np.float64)
    exact = _exact(x, w, b)
    bound = _gamma_bound(x, w) + (0 if b is None else 2.0 ** -23 * np.abs(b))
    # products carry at most 2^-22 relative error on the GPU (two f16 parts): both
    # sides sit within the f32 accumulation bound
    assert (np.abs(got - exact) <= bound).all()
    assert (np.abs(ref - exact) <= bound).all()
    assert (np.abs(got - ref) <= 2 * bound).all()


@pytest.mark.parametrize("n_tokens,n_in,n_out,x_dt,out_dt", [
    (1, 1280, 1280, "f32", torch.float32), (5, 1280, 5120, "f32", torch.float32),
    (8, 5120, 1280, "f32", torch.float32), (5, 1280, 51866, "f16", torch.float32),
    (3, 2112, 130, "f32", torch.bfloat16), (7, 4160, 1001, "f16", torch.float16)])
def test_decode_weight_stream(wrs, orc, ctx, n_tokens, n_in, n_out, x_dt, out_dt):
    """Decode-sized batches (quant.rs:392-413 / :434-437) on the weight-stream
    kernel: any n_out (the vocabulary is 51866), x chunks past 2048 columns."""
    note(f"gemv T={n_tokens} K={n_in} N={n_out} x={x_dt} out={out_dt}")
    rng = np.random.default_rng(n_in + n_out + n_tokens)
    x = rng.standard_normal((n_tokens, n_in)).astype(np.float32)
    if x_dt == "f16":
        x = x.astype(np.float16).astype(np.float32)
    w = _weights(n_out, n_in, n_out)
    b = rng.standard_normal(n_out).astype(np.float32)
    xd = dev(x) if x_dt == "f32" else torch.from_numpy(x).half().cuda()
    out = torch.full((n_tokens, n_out), float("nan"), dtype=out_dt, device="cuda")
    wrs.linear(xd, torch.from_numpy(w).cuda(), dev(b), out, ctx=ctx)
    got = out.float().cpu().numpy().astype(np.float64)
    ref = np.zeros(n_tokens * n_out, np.float32)
    orc.f16_linear(w, n_out, n_in, x.ravel(), b, n_tokens, ref)
    ref = ref.reshape(n_tokens, n_out)
    if out_dt == torch.float32:
        tol = 2 * (_gamma_bound(x, w) + 2.0 ** -23 * np.abs(b))
        assert (np.abs(got - ref) <= tol).all()
    else:
        rt = torch.from_numpy(ref).to(out_dt).float().numpy().astype(np.float64)
        tol = _rounded_tol(x, w, rt, "f16" if out_dt == torch.float16 else "bf16") + \
            2.0 ** -22 * np.abs(b)
        assert (np.abs(got - rt) <= tol).all()


@pytest.mark.parametrize("n_in", [256, 3200])
def test_linear_f32_row_scaling(wrs, orc, ctx, n_in):
    """Rows of very different magnitude (1e-30 .. 1e30, a zero row) stay exact:
    each row is scaled by a power of two before the f16 split (rows held in
    registers, and longer rows staged by the whole workgroup)."""
    note(f"linear f32 row scaling, {n_in} columns")
    n_out = 64
    rng = np.random.default_rng(11)
    x = rng.standard_normal((6, n_in)).astype(np.float32)
    x *= np.array([[1e-30], [1e-6], [1.0], [7e4], [1e30], [0.0]], np.float32)
    w = _weights(n_out, n_in, 12, scale=0.01)
    out = torch.zeros((6, n_out), device="cuda")
    wrs.linear(dev(x), torch.from_numpy(w).cuda(), None, out, ctx=ctx)
    got = host(out).astype(np.float64)
    exact = _exact(x, w, None)
    assert (np.abs(got - exact) <= _gamma_bound(x, w) + 1e-45).all()
    assert (got[5] == 0).all()


@pytest.mark.parametrize("out_dt", [torch.float32, torch.float16, torch.bfloat16])
def test_linear_f16_input_and_output_types(wrs, orc, ctx, out_dt):
    note(f"linear f16 x, out {out_dt}")
    n_tokens, n_in, n_out = 200, 384, 384
    rng = np.random.default_rng(21)
    x = rng.standard_normal((n_tokens, n_in)).astype(np.float16)
    w = _weights(n_out, n_in, 22)
    b = rng.standard_normal(n_out).astype(np.float32)
    out = torch.zeros((n_tokens, n_out), dtype=out_dt, device="cuda")
    wrs.linear(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), dev(b), out, ctx=ctx)
    got = out.float().cpu().numpy().astype(np.float64)
    ref = np.zeros(n_tokens * n_out, np.float32)
    orc.f16_linear(w, n_out, n_in, x.astype(np.float32).ravel(), b, n_tokens, ref)
    ref = ref.reshape(n_tokens, n_out)
    if out_dt == torch.float32:
        bound = 2 * (_gamma_bound(x, w) + 2.0 ** -23 * np.abs(b))
        assert (np.abs(got - ref) <= bound).all()
    else:
        # the f32 results round to the output type: at most one ulp apart
        rt = torch.from_numpy(ref).to(out_dt).float().numpy().astype(np.float64)
        tol = _rounded_tol(x, w, rt, "f16" if out_dt == torch.float16 else "bf16") + \
            2.0 ** -22 * np.abs(b)
        bad = np.argwhere(np.abs(got - rt) > tol)
        assert bad.size == 0, [(tuple(i), got[tuple(i)], rt[tuple(i)], ref[tuple(i)])
                               for i in bad[:8]]
        assert np.mean(got == rt) > 0.99


def test_linear_head_plane_layout(wrs, orc, ctx):
    """out(t, r) at t*64 + (r/64)*plane + r%64: the arena's [head][token][64]."""
    note("linear head-plane layout")
    n_tokens, n_in, n_out, plane_rows = 70, 256, 256, 96
    x = np.random.default_rng(31).standard_normal((n_tokens, n_in)).astype(np.float32)
    w = _weights(n_out, n_in, 32)
    out = torch.full((n_out // 64, plane_rows, 64), float("nan"), device="cuda")
    wrs.linear(dev(x), torch.from_numpy(w).cuda(), None, out, out_row_stride=64,
               out_head_stride=plane_rows * 64, ctx=ctx)
    got = host(out)
    ref = np.zeros(n_tokens * n_out, np.float32)
    orc.f16_linear(w, n_out, n_in, x.ravel(), None, n_tokens, ref)
    ref = ref.reshape(n_tokens, n_out // 64, 64).transpose(1, 0, 2)
    assert np.abs(got[:, :n_tokens] - ref).max() <= 1e-4
    assert np.isnan(got[:, n_tokens:]).all()  # rows past n_tokens untouched


@pytest.mark.parametrize("n_tokens,n_out,pad,offset,x_dt,out_dt", [
    (300, 260, 0, 0, "f16", torch.bfloat16),    # n_out % 8 == 4: last chunk is 8 bytes
    (300, 264, 8, 0, "f16", torch.float16),     # 16-byte rows, padded: pad untouched
    (513, 512, 4, 4, "f16", torch.bfloat16),    # 8-byte aligned start: 8-byte stores
    (257, 328, 0, 0, "f32", torch.float16),     # second feature tile 72 rows; row scales
    (323, 1284, 12, 0, "f32", torch.bfloat16),  # 6 feature tiles, 2 token tiles
])
def test_linear_16bit_output_edges(wrs, ctx, n_tokens, n_out, pad, offset, x_dt, out_dt):
    """16-bit output leaves the tile as whole token rows: the values equal the
    same launch's f32 output rounded to the output type, bit for bit (one
    accumulation, one rounding), at every alignment and partial edge, and
    nothing outside the written range changes."""
    note(f"linear 16-bit edges T={n_tokens} N={n_out} pad={pad} off={offset} x={x_dt} {out_dt}")
    n_in = 192
    rng = np.random.default_rng(n_tokens + n_out)
    xh = rng.standard_normal((n_tokens, n_in)).astype(np.float32)
    x = torch.from_numpy(xh if x_dt == "f32" else xh.astype(np.float16)).cuda()
    w = torch.from_numpy(_weights(n_out, n_in, n_out)).cuda()
    b = dev(rng.standard_normal(n_out).astype(np.float32))
    ref = torch.full((n_tokens, n_out), float("nan"), device="cuda")
    wrs.linear(x, w, b, ref, ctx=ctx)
    rs = n_out + pad
    buf = torch.full((offset + (n_tokens + 2) * rs,), float("nan"), dtype=out_dt, device="cuda")
    out = buf[offset:]
    wrs.linear(x, w, b, out, out_row_stride=rs, ctx=ctx)
    torch.cuda.synchronize()
    got = out[:n_tokens * rs].view(n_tokens, rs)
    want = ref.to(out_dt)
    assert torch.equal(got[:, :n_out].view(torch.int16), want.view(torch.int16))
    assert torch.isnan(got[:, n_out:].float()).all()
    assert torch.isnan(out[n_tokens * rs:].float()).all()
    assert torch.isnan(buf[:offset].float()).all()


def test_linear_16bit_head_planes(wrs, ctx):
    """16-bit output into [head][token][64] planes (the arena layout): equal to
    the same launch's f32 output rounded, rows past n_tokens untouched."""
    note("linear 16-bit head planes")
    n_tokens, n_in, n_out, plane_rows = 300, 128, 320, 304
    rng = np.random.default_rng(77)
    x = torch.from_numpy(rng.standard_normal((n_tokens, n_in)).astype(np.float16)).cuda()
    w = torch.from_numpy(_weights(n_out, n_in, 78)).cuda()
    ref = torch.full((n_out // 64, plane_rows, 64), float("nan"), device="cuda")
    wrs.linear(x, w, None, ref, out_row_stride=64, out_head_stride=plane_rows * 64, ctx=ctx)
    out = torch.full((n_out // 64, plane_rows, 64), float("nan"), dtype=torch.float16,
                     device="cuda")
    wrs.linear(x, w, None, out, out_row_stride=64, out_head_stride=plane_rows * 64, ctx=ctx)
    torch.cuda.synchronize()
    assert torch.equal(out[:, :n_tokens].view(torch.int16),
                       ref[:, :n_tokens].half().view(torch.int16))
    assert torch.isnan(out[:, n_tokens:].float()).all()


def test_linear_argument_errors(wrs, ctx):
    note("linear argument errors")
    w = torch.zeros((64, 96), dtype=torch.float16, device="cuda")
    x = torch.zeros((3, 96), device="cuda")
    with pytest.raises(RuntimeError):  # n_in not a multiple of 64
        wrs.linear(x, w, None, torch.zeros((3, 64), device="cuda"), ctx=ctx)
    with pytest.raises(AssertionError):  # W columns != x columns (quant.rs:440)
        wrs.linear(torch.zeros((3, 64), device="cuda"), w, None,
                   torch.zeros((3, 64), device="cuda"), ctx=ctx)
    # zero tokens: nothing written (quant.rs:430-432)
    o = torch.full((1, 64), 5.0, device="cuda")
    wrs.linear(torch.zeros((0, 64), device="cuda"), torch.zeros((64, 64), dtype=torch.float16,
               device="cuda"), None, o, ctx=ctx)
    assert float(o.min()) == 5.0


def test_fused_qkv_feeds_encoder_attention(wrs, orc, ctx):
    """encoder.rs:275-299: the fused QKV projection writes [t][3 d_model] bf16 rows
    that the encoder attention reads in place. The rows equal the oracle's
    f16_linear rounded to bf16 (one ulp where the f32 sums straddle a rounding
    boundary); the attention over them matches flash_attention_2 on the same
    bf16 values."""
    note("fused qkv -> prefill")
    T, H = 300, 4
    dm = 64 * H
    rng = np.random.default_rng(41)
    x = rng.standard_normal((T, dm)).astype(np.float32)
    w = _weights(3 * dm, dm, 42)
    b = (0.1 * rng.standard_normal(3 * dm)).astype(np.float32)
    qkv = torch.zeros((T, 3 * dm), dtype=torch.bfloat16, device="cuda")
    wrs.linear(dev(x), torch.from_numpy(w).cuda(), dev(b), qkv, ctx=ctx)
    lay = wrs.token_major(T, dm, 64, row_stride=3 * dm)
    olay = wrs.token_major(T, dm, 64)
    out = torch.full((T, dm), float("nan"), device="cuda")
    wrs.prefill(qkv[:, :dm], qkv[:, dm:2 * dm], qkv[:, 2 * dm:], out, batch=1, n_heads=H, t_q=T,
                t_kv=T, d_head=64, q_layout=lay, kv_layout=lay, out_layout=olay, ctx=ctx)
    got_qkv = qkv.float().cpu().numpy()
    ref_qkv = np.zeros(T * 3 * dm, np.float32)
    orc.f16_linear(w, 3 * dm, dm, x.ravel(), b, T, ref_qkv)
    rq = torch.from_numpy(ref_qkv.reshape(T, 3 * dm)).to(torch.bfloat16).float().numpy()
    tol = _rounded_tol(x, w, rq, "bf16") + 2.0 ** -22 * np.abs(b)
    assert (np.abs(got_qkv - rq) <= tol).all()
    assert np.mean(got_qkv == rq) > 0.99
    q, k, v = (np.ascontiguousarray(got_qkv[:, i * dm:(i + 1) * dm]) for i in range(3))
    ref = np.zeros(T * dm, np.float32)
    orc.flash_attention_2(q.ravel(), k.ravel(), v.ravel(), T, T, H, dm, False, ref)
    assert np.abs(host(out).ravel() - ref).max() <= TOL16


def test_cross_projection_into_arena(wrs, orc, ctx):
    """precompute_cross_attn (decoder.rs:423-447) straight into the f16 arena, every
    layer in one launch; planes equal the oracle's f32 K/V rounded to f16 (one
    ulp where the two f32 sums straddle a rounding boundary), and a cross decode
    over them matches attention over those K/V."""
    note("cross projection into arena")
    L, H, n_audio, n_max = 3, 4, 1500, 1504
    dm = 64 * H
    rng = np.random.default_rng(51)
    enc = rng.standard_normal((n_audio, dm)).astype(np.float32)
    wk = [_weights(dm, dm, 60 + l) for l in range(L)]
    wv = [_weights(dm, dm, 70 + l) for l in range(L)]
    bv = [(0.1 * rng.standard_normal(dm)).astype(np.float32) for _ in range(L)]
    arena = wrs.KvArena(L, 1, H, 448, n_max, ctx=ctx)
    arena.set_cross_proj(dev(enc), [torch.from_numpy(t).cuda() for t in wk],
                         [torch.from_numpy(t).cuda() for t in wv], [dev(t) for t in bv])
    torch.cuda.synchronize()
    assert arena.cross_len() == n_audio
    _, _, kc, vc = arena.plane_pointers()
    for l in (0, L - 1):
        for name, base, wt, bt in (("k", kc, wk[l], None), ("v", vc, wv[l], bv[l])):
            ref = np.zeros(n_audio * dm, np.float32)
            orc.f16_linear(wt, dm, dm, enc.ravel(), bt, n_audio, ref)
            ref16 = ref.reshape(n_audio, H, 64).transpose(1, 0, 2).astype(np.float16)
            for h in range(H):
                off = (l * H + h) * n_max * 64
                got = read_f16(base, off, n_audio * 64).reshape(n_audio, 64)
                r = ref16[h].astype(np.float32)
                xs = enc
                wh = wt[h * 64:(h + 1) * 64]
                tol = _rounded_tol(xs, wh, r, "f16")
                if bt is not None:
                    tol = tol + 2.0 ** -22 * np.abs(bt[h * 64:(h + 1) * 64])
                assert (np.abs(got - r) <= tol).all(), (name, l, h)
                assert np.mean(got == r) > 0.99
    # a cross decode over the projected planes
    q = rng.standard_normal((5, dm)).astype(np.float32)
    out = torch.zeros((5, dm), device="cuda")
    arena.decode_cross(L - 1, dev(q), out)
    kr = np.zeros(n_audio * dm, np.float32)
    vr = np.zeros(n_audio * dm, np.float32)
    orc.f16_linear(wk[L - 1], dm, dm, enc.ravel(), None, n_audio, kr)
    orc.f16_linear(wv[L - 1], dm, dm, enc.ravel(), bv[L - 1], n_audio, vr)
    ref = attention_f64(q, kr.reshape(n_audio, dm).astype(np.float16).astype(np.float32),
                        vr.reshape(n_audio, dm).astype(np.float16).astype(np.float32), 5,
                        n_audio, H, dm)
    assert np.abs(host(out) - ref).max() <= TOL16
    arena.close()


@pytest.mark.parametrize("n_tokens,x_dt", [(5, "f32"), (1, "f16"), (8, "f32"), (200, "f32"),
                                            (70, "f16")])
def test_linear_group_equals_separate_calls(wrs, ctx, n_tokens, x_dt):
    """The q, k, v projections of one input in one launch (decoder.rs:597-611)
    give bit-for-bit the outputs of three wrs_linear calls; the k projection
    has no bias, as in the reference."""
    note(f"linear group T={n_tokens} x={x_dt}")
    n_in, n_out = 384, 384
    rng = np.random.default_rng(n_tokens + 3)
    x = rng.standard_normal((n_tokens, n_in)).astype(np.float32)
    xd = dev(x) if x_dt == "f32" else torch.from_numpy(x).half().cuda()
    ws = [torch.from_numpy(_weights(n_out, n_in, 40 + i)).cuda() for i in range(3)]
    bs = [dev(rng.standard_normal(n_out).astype(np.float32)), None,
          dev(rng.standard_normal(n_out).astype(np.float32))]
    outs = [torch.full((n_tokens, n_out), float("nan"), device="cuda") for _ in range(3)]
    wrs.linear_group(xd, ws, bs, outs, ctx=ctx)
    for w, b, o in zip(ws, bs, outs):
        ref = torch.full((n_tokens, n_out), float("nan"), device="cuda")
        wrs.linear(xd, w, b, ref, ctx=ctx)
        assert torch.equal(o.cpu(), ref.cpu())


def test_linear_group_rejects_bad_arguments(wrs, ctx):
    note("linear group errors")
    x = torch.zeros((2, 64), device="cuda")
    w = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    short = torch.zeros((2, 32), device="cuda")
    with pytest.raises(AssertionError, match="shorter"):  # the reference asserts lengths
        wrs.linear_group(x, [w, w], None, [torch.zeros((2, 64), device="cuda"), short], ctx=ctx)


@pytest.mark.parametrize("n_tokens,n_groups,act,out_dt", [
    (5, 3, None, torch.float32), (1, 1, None, torch.float32), (2, 1, "gelu", torch.float32),
    (5, 1, "gelu", torch.float32), (8, 2, "gelu", torch.float16), (3, 1, None, torch.bfloat16),
    (40, 3, None, torch.float32), (40, 1, "gelu", torch.float32)])
def test_linear_fused_equals_unfused_calls(wrs, ctx, n_tokens, n_groups, act, out_dt):
    """layer_norm -> linear group -> gelu in one launch (decoder.rs:586-611,
    :737-753) gives bit for bit what wrs_layer_norm, wrs_linear_group and
    wrs_gelu_inplace give one after another (GELU in f32, then the output
    rounding); 40 rows take the batched path with the norm as its own launch."""
    note(f"linear fused T={n_tokens} groups={n_groups} act={act} out={out_dt}")
    n_in, n_out = 1280, 384
    rng = np.random.default_rng(n_tokens * 13 + n_groups)
    x = (2.0 * rng.standard_normal((n_tokens, n_in)) + 0.5).astype(np.float32)
    gamma = dev((1.0 + 0.1 * rng.standard_normal(n_in)).astype(np.float32))
    beta = dev((0.1 * rng.standard_normal(n_in)).astype(np.float32))
    ws = [torch.from_numpy(_weights(n_out, n_in, 70 + i)).cuda() for i in range(n_groups)]
    bs = [dev(rng.standard_normal(n_out).astype(np.float32)) if i % 2 == 0 else None
          for i in range(n_groups)]
    outs = [torch.full((n_tokens, n_out), float("nan"), dtype=out_dt, device="cuda")
            for _ in range(n_groups)]
    xd = dev(x)
    wrs.linear_fused(xd, ws, bs, outs, ln=(gamma, beta, 1e-5), act=act, ctx=ctx)
    normed = torch.empty((n_tokens, n_in), device="cuda")
    wrs.layer_norm(xd, gamma, beta, 1e-5, normed, ctx=ctx)
    for w, b, o in zip(ws, bs, outs):
        ref = torch.empty((n_tokens, n_out), device="cuda")
        wrs.linear(normed, w, b, ref, ctx=ctx)
        if act == "gelu":
            wrs.gelu_inplace(ref, ctx=ctx)
        assert torch.equal(o.cpu(), ref.to(out_dt).cpu())


def test_linear_fused_rejects_half_norm(wrs, ctx):
    note("linear fused errors")
    x = torch.zeros((2, 64), device="cuda")
    w = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    g = torch.ones(64, device="cuda")
    with pytest.raises(AssertionError, match="gamma and beta"):
        wrs._L.lib()  # the library loads
        ctx.check(wrs._L.lib().wrs_linear_fused(
            ctx.handle, x.data_ptr(), x.numel(), 64, g.data_ptr(), None, 1e-5, 1,
            (wrs.ctypes.c_void_p * 1)(w.data_ptr()), None, 2, 64, 64, 0, 0,
            (wrs.ctypes.c_void_p * 1)(torch.zeros((2, 64), device="cuda").data_ptr()),
            (wrs.ctypes.c_size_t * 1)(128), 64, 64), "linear_fused")
