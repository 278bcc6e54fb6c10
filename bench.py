"""Benchmark of the whisper.rs attention path on one MI355X.

Headline workload (``value``): whisper-large-v3 encoder self-attention,
16 windows x 20 heads x 1500 frames x d_head 64, bf16 Q/K/V ~ N(0, 0.5^2)
with 13 outlier channels x8, f32 accumulate -- one step is one prefill launch
over all 16 windows, inputs resident in HBM. FLOPs are 4*B*H*T^2*d (the
reference's convention, crates/tensor/tests/bench_flash_attention_tiled.rs:214).

Second figure of the same metric (``decode_cross``): whisper-large-v3
cross-attention decode, beam 5 x 20 heads against 1500 f16 encoder K/V per
layer, 32 layers resident, one launch per layer. Three utterances' caches
(737 MB) are rotated so the 256 MB MALL cannot hold them; the launches are
replayed from a HIP graph. Bytes are the unique K/V bytes (read once for all
beams) plus f32 Q and O.

cpu_baseline: the CPU oracle (a C restatement of the reference path) timed on
this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import shutil
import sqlite3
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
METRIC = "encoder attn TFLOP/s (%MFMA peak) + decode cross-attn GB/s (%HBM), large-v3"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E


def _load_pkg():
    pkg_dir = ROOT / "whisper.rs_amd"
    spec = importlib.util.spec_from_file_location(
        "wrs_amd", pkg_dir / "__init__.py", submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["wrs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bench_encoder(wrs, W, ctx, steps, warmup):
    import torch
    cfg = W.LARGE_ENCODER
    log(f"encoder: generating {cfg.name}")
    q, k, v = cfg.inputs()
    qd, kd, vd = (torch.from_numpy(x).to(torch.bfloat16).cuda() for x in (q, k, v))
    B, T, dm = cfg.batch, cfg.t, cfg.d_model
    out = torch.empty((B, T, dm), dtype=torch.float32, device="cuda")
    lay = wrs.token_major(T, dm, 64)

    def step():
        wrs.prefill(qd, kd, vd, out, batch=B, n_heads=cfg.n_heads, t_q=T, t_kv=T, d_head=64,
                    q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)

    log(f"encoder: warmup {warmup}")
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"encoder: timing {steps} steps")
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tflops = cfg.flops() / (ms * 1e-3) / 1e12
    return cfg, ms, tflops, (q, k, v)


def bench_decode(wrs, W, ctx, reps, use_graph=True):
    import torch
    cfg = W.LARGE_CROSS_DECODE
    U = 3  # utterances rotated: 3 x 245.76 MB of cross K/V > 256 MB MALL
    log(f"decode: building {U} x {cfg.n_layers}-layer cross caches")
    arenas = []
    for u in range(U):
        ar = wrs.KvArena(cfg.n_layers, 1, cfg.n_heads, 448, cfg.n_audio, ctx=ctx)
        for layer in range(cfg.n_layers):
            kk, vv = cfg.kv(layer)
            ar.set_cross(layer, torch.from_numpy(kk).cuda(), torch.from_numpy(vv).cuda())
        arenas.append(ar)
    qs = torch.from_numpy(np.stack([cfg.q(layer) for layer in range(cfg.n_layers)])).cuda()
    outs = torch.zeros((U, cfg.n_layers, cfg.beams, cfg.d_model), device="cuda")

    def all_layers():
        for u in range(U):
            for layer in range(cfg.n_layers):
                arenas[u].decode_cross(layer, qs[layer], outs[u, layer])

    all_layers()  # sizes the scratch outside any capture
    torch.cuda.synchronize()
    if not use_graph:  # eager launches (counter passes)
        for _ in range(reps):
            all_layers()
        torch.cuda.synchronize()
        for ar in arenas:
            ar.close()
        return cfg, float("nan"), float("nan")
    eager = outs.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        all_layers()
    ctx.use_torch_stream()
    outs.zero_()
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(outs, eager):
        raise RuntimeError("graph replay of the decode launches differs from eager")
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"decode: timing {reps} graph replays of {U * cfg.n_layers} launches")
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    n_launch = reps * U * cfg.n_layers
    us = start.elapsed_time(end) * 1e3 / n_launch
    gbs = cfg.bytes_per_layer() / (us * 1e-6) / 1e9
    for ar in arenas:
        ar.close()
    return cfg, us, gbs


def bench_decode_self(wrs, W, ctx, reps):
    """Causal self-attention decode, whisper-small shape (beam 5 slots, 12 heads,
    valid length 224 of 448): one launch per layer over 12 layers, 8 arenas rotated
    so that the 330 MB read per round trip is larger than the 256 MB MALL."""
    import torch
    cfg = W.SMALL_SELF_DECODE
    n_layers, U = 12, 8
    log(f"decode self: building {U} x {n_layers}-layer self caches, length {cfg.ctx}")
    kvs = [cfg.kv(s) for s in range(cfg.beams)]
    kd = [(torch.from_numpy(k.astype(np.float32)).cuda(), torch.from_numpy(v.astype(np.float32)).cuda())
          for k, v in kvs]
    arenas = []
    for u in range(U):
        ar = wrs.KvArena(n_layers, cfg.beams, cfg.n_heads, cfg.max_ctx, 0, ctx=ctx)
        for s_ in range(cfg.beams):
            k, v = kd[s_]
            for layer in range(n_layers):
                ar.append(layer, s_, k[:cfg.ctx - 1], v[:cfg.ctx - 1])
            ar.advance(s_, cfg.ctx - 1)
            for layer in range(n_layers):
                ar.append(layer, s_, k[cfg.ctx - 1:], v[cfg.ctx - 1:])
        arenas.append(ar)
    q = torch.from_numpy(cfg.q()).cuda()
    outs = torch.zeros((U, n_layers, cfg.beams, cfg.d_model), device="cuda")
    slots = list(range(cfg.beams))

    def all_layers():
        for u in range(U):
            for layer in range(n_layers):
                arenas[u].decode_self(layer, slots, q, outs[u, layer])

    all_layers()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        all_layers()
    ctx.use_torch_stream()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / (reps * U * n_layers)
    for ar in arenas:
        ar.close()
    return cfg, us, cfg.bytes() / (us * 1e-6) / 1e9


def bench_capture(wrs, W, ctx, reps, use_graph=True):
    """DTW alignment pass: one capture launch per preset layer, inputs resident."""
    import torch
    cfg = W.LARGE_DTW_CAPTURE
    layers = cfg.layers()
    ar = wrs.KvArena(cfg.n_layers, 1, cfg.n_heads, 448, cfg.n_audio, ctx=ctx)
    zeros = torch.zeros((cfg.n_audio, cfg.d_model), device="cuda")
    for layer in layers:
        ar.set_cross(layer, torch.from_numpy(cfg.k(layer)).cuda(), zeros)
    qs = {layer: torch.from_numpy(cfg.q(layer)).cuda() for layer in layers}
    n_sel = len(cfg.heads)
    out = torch.zeros(cfg.n_tokens * n_sel * cfg.n_audio, device="cuda")

    def all_layers():
        for layer in layers:
            ar.capture_cross_heads(layer, qs[layer], cfg.pairs(layer), n_sel, 0, out)

    all_layers()
    torch.cuda.synchronize()
    if not use_graph:
        for _ in range(reps):
            all_layers()
        torch.cuda.synchronize()
        ar.close()
        return cfg, float("nan"), float("nan")
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        all_layers()
    ctx.use_torch_stream()
    out.zero_()
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(out, eager):
        raise RuntimeError("graph replay of the capture launches differs from eager")
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"capture: timing {reps} graph replays of {len(layers)} launches")
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / (reps * len(layers))
    gbs = cfg.bytes_per_pair() / (us * 1e-6) / 1e9  # one pair per preset layer
    ar.close()
    return cfg, us, gbs


def bench_linear(wrs, cfg, ctx, reps):
    """One fused QKV projection per step, inputs resident; bf16 rows out."""
    import torch
    x = torch.from_numpy(cfg.x()).cuda()
    if cfg.x_storage == "f16":
        x = x.half()
    w = torch.from_numpy(cfg.w()).cuda()
    b = torch.from_numpy(cfg.bias()).cuda()
    out = torch.empty((cfg.n_tokens, cfg.n_out), dtype=torch.bfloat16, device="cuda")
    for _ in range(150):  # ~50 ms of work: the clocks settle first
        wrs.linear(x, w, b, out, ctx=ctx)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"linear: timing {reps} launches ({cfg.name})")
    start.record()
    for _ in range(reps):
        wrs.linear(x, w, b, out, ctx=ctx)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    return ms, cfg.flops() / (ms * 1e-3) / 1e12


def bench_weight_stream(wrs, W, ctx, reps):
    """One decoder step's projections for 5 beams, replayed from a HIP graph:
    every launch streams its f16 weights once (the decode-sized linear path)."""
    import torch
    cfg = W.LARGE_DECODE_WEIGHTS
    gen = torch.Generator(device="cuda").manual_seed(0x5EED)
    mats = cfg.matrices()
    shapes = sorted(set(mats))
    weights = {}
    for r, c in shapes:
        n = sum(1 for m in mats if m == (r, c))
        weights[(r, c)] = [(torch.randn((r, c), generator=gen, device="cuda") * c ** -0.5).half()
                           for _ in range(n)]
    xs = {c: torch.randn((cfg.beams, c), generator=gen, device="cuda") for _, c in shapes}
    outs = {r: torch.empty((cfg.beams, r), device="cuda") for r, _ in shapes}
    seq, used = [], {k: 0 for k in shapes}
    for m in mats:
        seq.append((xs[m[1]], weights[m][used[m]], outs[m[0]]))
        used[m] += 1
    # Each layer's self-attention q, k, v share their input (decoder.rs:597-611):
    # one grouped launch; the other projections are one launch each.
    per_layer = len(mats[:-1]) // cfg.n_layers
    qkv_outs = [torch.empty((cfg.beams, cfg.d_model), device="cuda") for _ in range(3)]
    calls = []
    for layer in range(cfg.n_layers):
        first = layer * per_layer
        x0 = seq[first][0]
        calls.append(("group", x0, [seq[first + i][1] for i in range(3)], qkv_outs))
        for x, w, o in seq[first + 3:first + per_layer]:
            calls.append(("one", x, w, o))
    calls.append(("one",) + seq[-1])

    def step():
        for kind, x, w, o in calls:
            if kind == "group":
                wrs.linear_group(x, w, None, o, ctx=ctx)
            else:
                wrs.linear(x, w, None, o, ctx=ctx)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        step()
    ctx.use_torch_stream()
    for _ in range(5):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"weight stream: timing {reps} graph replays of {len(calls)} launches")
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    # The same step with its LayerNorms (decoder.rs:586-594, :660-668, :737-745, the
    # final one before the vocabulary), the MLP GELU (:753) and the biases the
    # reference's projections carry (q, v, out, cross q, cross out, mlp0, mlp2; k and the
    # vocabulary have none): as separate launches, then fused into the projections
    # (wrs_linear_fused).
    d = cfg.d_model
    bd = torch.randn(d, generator=gen, device="cuda") * 0.1
    b4d = torch.randn(4 * d, generator=gen, device="cuda") * 0.1
    lng = torch.randn(d, generator=gen, device="cuda") * 0.1 + 1.0
    lnb = torch.randn(d, generator=gen, device="cuda") * 0.1
    normed = torch.empty((cfg.beams, d), device="cuda")
    xres = xs[d]
    hid = outs[4 * d]
    wl = [seq[i][1] for i in range(len(seq))]

    def layer_weights(layer):
        first = layer * per_layer
        return wl[first:first + per_layer]

    def step_unfused():
        for layer in range(cfg.n_layers):
            q, k, v, o, cq, co, m0, m2 = layer_weights(layer)
            wrs.layer_norm(xres, lng, lnb, 1e-5, normed, ctx=ctx)
            wrs.linear_group(normed, [q, k, v], [bd, None, bd], qkv_outs, ctx=ctx)
            wrs.linear(xres, o, bd, outs[d], ctx=ctx)
            wrs.layer_norm(xres, lng, lnb, 1e-5, normed, ctx=ctx)
            wrs.linear(normed, cq, bd, outs[d], ctx=ctx)
            wrs.linear(xres, co, bd, outs[d], ctx=ctx)
            wrs.layer_norm(xres, lng, lnb, 1e-5, normed, ctx=ctx)
            wrs.linear(normed, m0, b4d, hid, ctx=ctx)
            wrs.gelu_inplace(hid, ctx=ctx)
            wrs.linear(hid, m2, bd, outs[d], ctx=ctx)
        wrs.layer_norm(xres, lng, lnb, 1e-5, normed, ctx=ctx)
        wrs.linear(normed, wl[-1], None, outs[cfg.n_vocab], ctx=ctx)

    def step_fused():
        ln = (lng, lnb, 1e-5)
        for layer in range(cfg.n_layers):
            q, k, v, o, cq, co, m0, m2 = layer_weights(layer)
            wrs.linear_fused(xres, [q, k, v], [bd, None, bd], qkv_outs, ln=ln, ctx=ctx)
            wrs.linear(xres, o, bd, outs[d], ctx=ctx)
            wrs.linear_fused(xres, [cq], [bd], [outs[d]], ln=ln, ctx=ctx)
            wrs.linear(xres, co, bd, outs[d], ctx=ctx)
            wrs.linear_fused(xres, [m0], [b4d], [hid], ln=ln, act="gelu", ctx=ctx)
            wrs.linear(hid, m2, bd, outs[d], ctx=ctx)
        wrs.linear_fused(xres, [wl[-1]], None, [outs[cfg.n_vocab]], ln=ln, ctx=ctx)

    norms = {}
    for name, fn, launches in (("unfused", step_unfused, cfg.launches() + 4 * cfg.n_layers + 1),
                               ("fused", step_fused, cfg.launches())):
        fn()
        torch.cuda.synchronize()
        gn = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gn):
            ctx.use_torch_stream()
            fn()
        ctx.use_torch_stream()
        for _ in range(3):
            gn.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            gn.replay()
        end.record()
        torch.cuda.synchronize()
        norms[name] = {"ms_per_step": round(start.elapsed_time(end) / reps, 4),
                       "launches_per_step": launches}
        log(f"weight stream with norms, {name}: {norms[name]['ms_per_step']} ms, "
            f"{launches} launches")
    # the vocabulary projection alone (the largest single stream)
    xv, wv, ov = seq[-1]
    for _ in range(10):
        wrs.linear(xv, wv, None, ov, ctx=ctx)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        wrs.linear(xv, wv, None, ov, ctx=ctx)
    end.record()
    torch.cuda.synchronize()
    ms_vocab = start.elapsed_time(end) / reps
    vocab_bytes = cfg.n_vocab * cfg.d_model * 2
    return cfg, ms, cfg.weight_bytes() / (ms * 1e-3) / 1e9, ms_vocab, \
        vocab_bytes / (ms_vocab * 1e-3) / 1e9, norms


def bench_rows(wrs, ctx, reps):
    """LayerNorm over the large-v3 encoder rows of 16 windows (24000 x 1280 f32
    in, bf16 out, encoder.rs:266-274) and GELU over their MLP activations
    (24000 x 5120 f32 in place): HBM-bound, algorithmic bytes = one read and
    one write."""
    import torch
    gen = torch.Generator(device="cuda").manual_seed(0x5EED)
    T, d = 24000, 1280
    x = torch.randn((T, d), generator=gen, device="cuda")
    g = torch.randn(d, generator=gen, device="cuda")
    b = torch.randn(d, generator=gen, device="cuda")
    y = torch.empty((T, d), dtype=torch.bfloat16, device="cuda")
    h = torch.randn((T, 4 * d), generator=gen, device="cuda")
    res = {}
    for name, fn, nbytes in (("layer_norm", lambda: wrs.layer_norm(x, g, b, 1e-5, y, ctx=ctx),
                              T * d * (4 + 2)),
                             ("gelu", lambda: wrs.gelu_inplace(h, ctx=ctx), T * 4 * d * 8)):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": round(ms, 4), "GBps": round(gbs, 1), "bytes": nbytes,
                     "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"rows: {name}: {ms:.4f} ms, {gbs:.1f} GB/s")
    return res


def bench_host_slice(wrs, W, ctx, reps=20):
    """The host-slice drop-in (flash_attention_2 on f32 host slices, PCIe both
    ways) against the same call on device-resident f32 tensors, whisper-tiny
    encoder shape. Informational: never the headline value."""
    import torch
    cfg = W.TINY_ENCODER
    q, k, v = (np.ascontiguousarray(x[0]) for x in cfg.inputs())
    out = np.empty_like(q)
    T, H, dm = cfg.t, cfg.n_heads, cfg.d_model
    for _ in range(3):
        wrs.flash_attention_2(q, k, v, T, T, H, dm, False, out, ctx=ctx)
    t0 = time.perf_counter()
    for _ in range(reps):
        wrs.flash_attention_2(q, k, v, T, T, H, dm, False, out, ctx=ctx)
    host_ms = (time.perf_counter() - t0) * 1e3 / reps
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    od = torch.empty_like(qd)
    lay = wrs.token_major(T, dm, 64)
    run = lambda: wrs.prefill(qd, kd, vd, od, batch=1, n_heads=H, t_q=T, t_kv=T, d_head=64,
                              q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
    for _ in range(20):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    e1.synchronize()
    dev_ms = e0.elapsed_time(e1) / reps
    gflop = cfg.flops() / 1e9
    return {"workload": cfg.name, "unit": "GFLOP/s",
            "host_slice_ms": round(host_ms, 3), "host_slice_value": round(gflop / host_ms * 1e3, 1),
            "device_resident_ms": round(dev_ms, 4),
            "device_resident_value": round(gflop / dev_ms * 1e3, 1),
            "pcie_bytes_per_call": 4 * q.nbytes}


def copy_bandwidth():
    import torch
    n = 1 << 28  # 1 GiB of f32
    a = torch.empty(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(10):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / 10
    return 2 * a.numel() * 4 / (ms * 1e-3) / 1e9


CALIB_BYTES = 256 << 20  # one plain device copy of this many bytes per profiled run


def calibration_copy():
    """A plain copy of known size: the reference point for FETCH_SIZE/WRITE_SIZE."""
    import torch
    a = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


def measure_traffic(only: str, kernel_tag: str, extra: list[str]):
    """HBM bytes per call of the kernel(s) whose name contains kernel_tag.

    Two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch)
    over `bench.py --only <only>`; each counter is scaled by what it reads for
    the plain copy of CALIB_BYTES in the same run. Returns None when rocprofv3
    is unavailable or a pass fails.
    """
    if shutil.which("rocprofv3") is None:
        return None
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory(dir="/tmp") as d:
            cmd = ["timeout", "-s", "KILL", "150", "rocprofv3", "--pmc", counter, "-d", d, "-o",
                   "t", "--", sys.executable, str(Path(__file__).resolve()), "--only", only] + extra
            env = dict(os.environ, TMPDIR="/tmp")
            r = subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, env=env,
                               cwd="/tmp")
            dbs = list(Path(d).rglob("*_results.db"))
            if r.returncode != 0 or not dbs:
                log(f"traffic: {counter} pass failed (rc={r.returncode})")
                return None
            db = sqlite3.connect(str(dbs[0]))
            rows = db.execute("select kernel_name, avg(value), max(value) from counters_collection "
                              "where counter_name = ? group by kernel_name", (counter,)).fetchall()
            db.close()
            kern = [v for n, v, _ in rows if kernel_tag in n]
            # the calibration copy is the largest dispatch of its kernel: other,
            # smaller copies (input set-up) can share the kernel's name
            copy = [vmax for n, _, vmax in rows if "copy" in n.lower() or "elementwise" in n.lower()]
            if not kern or not copy or max(copy) <= 0:
                log(f"traffic: {counter}: kernels not found in the profile")
                return None
            factor = CALIB_BYTES / (max(copy) * 1024.0)
            # one call of the path = one dispatch of each matching kernel
            # (the capture runs as two passes)
            out[counter] = sum(kern) * 1024.0 * factor
            out[counter + "_factor"] = factor
            log(f"traffic: {only} {counter} = {sum(kern):.1f} KiB per call over {len(kern)} "
                f"kernel(s), copy of {CALIB_BYTES} B reads {max(copy):.1f} KiB -> "
                f"factor {factor:.4f}")
    return out


def cpu_baseline_encoder(cfg, qkv, threads):
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    q, k, v = (np.ascontiguousarray(x[0].reshape(-1)) for x in qkv)
    out = np.zeros_like(q)
    T, H, dm = cfg.t, cfg.n_heads, cfg.d_model
    best = float("inf")
    t_end = time.time() + 20.0
    reps = 0
    while reps < 5 and (reps < 2 or time.time() < t_end):
        t0 = time.perf_counter()
        orc.flash_attention_2(q, k, v, T, T, H, dm, False, out, n_threads=threads)
        best = min(best, time.perf_counter() - t0)
        reps += 1
    flops = 4.0 * H * T * T * 64
    return {"value": flops / best / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"1 of 16 windows (20 heads x 1500 x 1500), best of {reps}, "
                      f"{best * 1e3:.1f} ms"}


def cpu_baseline_decode(cfg):
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    kk, vv = cfg.kv(0)
    k, v = np.ascontiguousarray(kk.ravel()), np.ascontiguousarray(vv.ravel())
    q = cfg.q(0)
    out = np.zeros(cfg.d_model, np.float32)
    best = float("inf")
    for _ in range(5):
        t0 = time.perf_counter()
        for b in range(cfg.beams):  # the reference's per-slot loop (decoder.rs:689-724)
            orc.single_token_mha_d64(np.ascontiguousarray(q[b]), k, v, cfg.n_audio, cfg.n_heads,
                                     cfg.d_model, out)
        best = min(best, time.perf_counter() - t0)
    return {"value": cfg.bytes_per_layer() / best / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"1 layer, 5 beams read serially from f32 K/V, best of 5, "
                      f"{best * 1e3:.2f} ms"}


def cpu_baseline_capture(cfg):
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    layer = cfg.layers()[0]
    q = np.ascontiguousarray(cfg.q(layer).ravel())
    k = np.ascontiguousarray(cfg.k(layer).ravel())
    sel = cfg.pairs(layer)
    out = np.zeros(cfg.n_tokens * len(cfg.heads) * cfg.n_audio, np.float32)
    best = float("inf")
    for _ in range(5):
        t0 = time.perf_counter()
        orc.capture_cross_attention_heads(q, k, cfg.n_tokens, cfg.n_audio, cfg.n_heads,
                                          cfg.d_model, sel, len(cfg.heads), 0, out)
        best = min(best, time.perf_counter() - t0)
    return {"value": cfg.bytes_per_pair() / best / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"1 layer's pair ({cfg.n_tokens} tokens x {cfg.n_audio} frames), best of 5, "
                      f"{best * 1e3:.2f} ms"}


def cpu_baseline_linear(cfg, threads):
    """The oracle's f16_linear on one 1500-frame window of the batch."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    n = 1500
    x = np.ascontiguousarray(cfg.x()[:n].astype(np.float32).ravel())
    w = np.ascontiguousarray(cfg.w())
    b = cfg.bias()
    out = np.zeros(n * cfg.n_out, np.float32)
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        orc.f16_linear(w, cfg.n_out, cfg.n_in, x, b, n, out, n_threads=threads)
        best = min(best, time.perf_counter() - t0)
    flops = 2.0 * n * cfg.n_in * cfg.n_out
    return {"value": flops / best / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"1 window of 16 ({n} x {cfg.n_in} x {cfg.n_out}), best of 3, "
                      f"{best * 1e3:.1f} ms"}


def cpu_baseline_stream(cfg, threads):
    """The oracle's f16_linear over one decoder layer's projections for the
    step's beams (q, k, v, out, cross q, cross out, mlp0, mlp2): f16 weights
    streamed once per matrix, as f16_gemv_parallel does (quant.rs:392-413)."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    rng = np.random.default_rng(0x5EED)
    mats = cfg.matrices()[:len(cfg.matrices()[:-1]) // cfg.n_layers]
    ws = [(rng.standard_normal((r, c)) * c ** -0.5).astype(np.float16) for r, c in mats]
    xs = {c: np.ascontiguousarray(rng.standard_normal((cfg.beams, c)).astype(np.float32).ravel())
          for _, c in mats}
    outs = {r: np.zeros(cfg.beams * r, np.float32) for r, _ in mats}
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        for w in ws:
            r, c = w.shape
            orc.f16_linear(w, r, c, xs[c], None, cfg.beams, outs[r], n_threads=threads)
        best = min(best, time.perf_counter() - t0)
    nbytes = sum(r * c * 2 for r, c in mats)
    return {"value": round(nbytes / best / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"one layer's 8 projections ({nbytes / 1e6:.1f} MB of f16 weights, "
                      f"{cfg.beams} rows), best of 3, {best * 1e3:.2f} ms"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # ~75 ms of untimed encoder steps: the clocks settle within about 300 steps
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--decode-reps", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--eager", action="store_true",
                    help="with --only decode: plain launches instead of a graph replay")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 HBM-traffic passes")
    ap.add_argument("--capture-reps", type=int, default=100)
    ap.add_argument("--linear-reps", type=int, default=50)
    ap.add_argument("--linear-f16-only", action="store_true",
                    help="with --only linear: the f16-activation projection only")
    ap.add_argument("--stream-reps", type=int, default=20)
    ap.add_argument("--rows-reps", type=int, default=50)
    ap.add_argument("--only", choices=["encoder", "decode", "capture", "linear", "stream", "rows"],
                    default=None,
                    help="run one workload only (for profiling); prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the attention path shards across GPUs by window, utterance or head, "
              "without exchange)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    wrs = _load_pkg()
    from wrs_amd import workloads as W
    ctx = wrs.Context(0)
    ctx.use_torch_stream()
    props = torch.cuda.get_device_properties(0)

    if args.only == "encoder":
        _, ms, tflops, _ = bench_encoder(wrs, W, ctx, args.steps, args.warmup)
        calibration_copy()
        log(f"encoder only: {ms:.4f} ms/step, {tflops:.1f} TFLOP/s")
        return
    if args.only == "decode":
        _, us, gbs = bench_decode(wrs, W, ctx, args.decode_reps, use_graph=not args.eager)
        calibration_copy()
        log(f"decode only: {us:.3f} us/launch, {gbs:.1f} GB/s")
        if not args.eager:
            _, sus, sgbs_ = bench_decode_self(wrs, W, ctx, args.decode_reps)
            log(f"decode self (whisper-small, length 224): {sus:.3f} us/launch, {sgbs_:.1f} GB/s")
        return
    if args.only == "linear":
        cfgs = (W.LARGE_QKV_F16,) if args.linear_f16_only else (W.LARGE_QKV_F16, W.LARGE_QKV_F32)
        for cfg in cfgs:
            lms, ltf = bench_linear(wrs, cfg, ctx, args.linear_reps)
            log(f"linear only: {cfg.name}: {lms:.4f} ms, {ltf:.1f} TFLOP/s")
        calibration_copy()
        return
    if args.only == "rows":
        bench_rows(wrs, ctx, args.rows_reps)
        calibration_copy()
        return
    if args.only == "stream":
        _, sms, sgbs, vms, vgbs, snorms = bench_weight_stream(wrs, W, ctx, args.stream_reps)
        calibration_copy()
        log(f"stream only: step {sms:.3f} ms, {sgbs:.1f} GB/s; vocabulary {vms * 1e3:.1f} us, "
            f"{vgbs:.1f} GB/s")
        return
    if args.only == "capture":
        _, cus, cgbs = bench_capture(wrs, W, ctx, args.capture_reps, use_graph=not args.eager)
        calibration_copy()
        log(f"capture only: {cus:.3f} us/launch, {cgbs:.1f} GB/s")
        return
    cfg, ms, tflops, qkv = bench_encoder(wrs, W, ctx, args.steps, args.warmup)
    dcfg, us, gbs = bench_decode(wrs, W, ctx, args.decode_reps)
    dscfg, dsus, dsgbs = bench_decode_self(wrs, W, ctx, args.decode_reps)
    ccfg, cus, cgbs = bench_capture(wrs, W, ctx, args.capture_reps)
    lcfg = W.LARGE_QKV_F16
    lms, ltf = bench_linear(wrs, lcfg, ctx, args.linear_reps)
    lms32, ltf32 = bench_linear(wrs, W.LARGE_QKV_F32, ctx, args.linear_reps)
    scfg, sms, sgbs, vms, vgbs, snorms = bench_weight_stream(wrs, W, ctx, args.stream_reps)
    rows = bench_rows(wrs, ctx, args.rows_reps)
    log("host-slice drop-in: whisper-tiny encoder, f32 host slices")
    host_slice = bench_host_slice(wrs, W, ctx)
    copy_gbs = copy_bandwidth()

    enc_traffic = dec_traffic = cap_traffic = lin_traffic = None
    if not args.no_traffic:
        log("traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE passes")
        enc_traffic = measure_traffic("encoder", "fa2_prefill", ["--steps", "3", "--warmup", "1"])
        dec_traffic = measure_traffic("decode", "decode_f16", ["--decode-reps", "3", "--eager"])
        cap_traffic = measure_traffic("capture", "capture_cross", ["--capture-reps", "3",
                                                                    "--eager"])
        lin_traffic = measure_traffic("linear", "linear_f16w",
                                      ["--linear-reps", "3", "--linear-f16-only"])

    def traffic_bytes(t):
        return None if t is None else round(t["FETCH_SIZE"] + t["WRITE_SIZE"])

    threads = min(16, os.cpu_count() or 1)
    cpu_enc = cpu_dec = cpu_cap = cpu_lin = cpu_stream = None
    if not args.no_cpu:
        log(f"cpu baseline: oracle encoder window on {threads} threads")
        cpu_enc = cpu_baseline_encoder(cfg, qkv, threads)
        log("cpu baseline: oracle decode layer, 1 thread")
        cpu_dec = cpu_baseline_decode(dcfg)
        log("cpu baseline: oracle capture of one layer, 1 thread")
        cpu_cap = cpu_baseline_capture(ccfg)
        log(f"cpu baseline: oracle f16_linear, one window, {threads} threads")
        cpu_lin = cpu_baseline_linear(lcfg, threads)
        log(f"cpu baseline: oracle f16_linear, one decoder layer's projections, {threads} threads")
        cpu_stream = cpu_baseline_stream(scfg, threads)

    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": cfg.name, "windows": cfg.batch, "heads": cfg.n_heads,
                   "frames": cfg.t, "d_head": 64, "flops_per_step": cfg.flops()},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_bytes(enc_traffic)},
        "cpu_baseline": cpu_enc,
        "decode_cross": {
            "workload": dcfg.name, "value": round(gbs, 1), "unit": "GB/s",
            "us_per_launch": round(us, 3), "launches_per_step": dcfg.n_layers,
            "bytes_per_launch": dcfg.bytes_per_layer(), "dtype": "f16",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic_bytes(dec_traffic)},
            "cpu_baseline": cpu_dec,
        },
        "decode_self": {
            "workload": dscfg.name + f", valid length {dscfg.ctx} of {dscfg.max_ctx}",
            "value": round(dsgbs, 1), "unit": "GB/s", "us_per_launch": round(dsus, 3),
            "launches_per_step": 12, "bytes_per_launch": dscfg.bytes(), "dtype": "f16",
            "roofline": {"bound": "hbm", "achieved": round(dsgbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(dsgbs / PEAK_HBM_GBS, 4),
                         "traffic": None},
        },
        "capture": {
            "workload": ccfg.name, "value": round(cgbs, 1), "unit": "GB/s",
            "us_per_launch": round(cus, 3), "launches_per_step": len(ccfg.layers()),
            "bytes_per_launch": ccfg.bytes_per_pair(), "dtype": "f32",
            "roofline": {"bound": "hbm", "achieved": round(cgbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(cgbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic_bytes(cap_traffic)},
            "cpu_baseline": cpu_cap,
        },
        "projection": {
            "workload": lcfg.name, "value": round(ltf, 2), "unit": "TFLOP/s",
            "ms_per_launch": round(lms, 4), "flops_per_launch": lcfg.flops(), "dtype": "f16",
            "roofline": {"bound": "mfma", "achieved": round(ltf, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ltf / PEAK_BF16_TFLOPS, 4),
                         "traffic": traffic_bytes(lin_traffic)},
            "f32_exact": {"workload": W.LARGE_QKV_F32.name, "value": round(ltf32, 2),
                          "unit": "TFLOP/s", "ms_per_launch": round(lms32, 4)},
            "cpu_baseline": cpu_lin,
        },
        "decoder_weight_stream": {
            "workload": scfg.name, "value": round(sgbs, 1), "unit": "GB/s",
            "ms_per_step": round(sms, 4), "launches_per_step": scfg.launches(),
            "weight_bytes_per_step": scfg.weight_bytes(), "dtype": "f16",
            "roofline": {"bound": "hbm", "achieved": round(sgbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(sgbs / PEAK_HBM_GBS, 4), "traffic": None},
            "vocabulary_projection": {"us": round(vms * 1e3, 2), "GBps": round(vgbs, 1),
                                      "frac_hbm": round(vgbs / PEAK_HBM_GBS, 4)},
            "with_layer_norms_and_gelu": snorms,
            "cpu_baseline": cpu_stream,
        },
        "row_kernels": rows,
        "host_slice": host_slice,
        "device": {"name": props.name, "cu": props.multi_processor_count,
                   "copy_GBps": round(copy_gbs, 1)},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
