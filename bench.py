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

Timing: each timed encoder leg first runs a time-bounded clock-settle phase
(SETTLE_SECONDS of the same launch, reported in the line's config), then
`--warmup` untimed steps, then `--steps` timed steps. Decode legs replay HIP
graphs of one launch per layer and divide by the launch count.

cpu_baseline: the CPU oracle (a C restatement of the reference path) timed on
this host on a bounded sample, by the reference's own benchmark method
(best of 9 after a warm call; encoder legs alternate the tiled kernel with the
materialized baseline on available_parallelism() threads).
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


SETTLE_SECONDS = 1.5  # clock-settle phase before the timed encoder steps


def settle_clocks(fn, seconds: float = SETTLE_SECONDS) -> int:
    """Run `fn` (one launch of the timed workload) for `seconds` of wall time.

    MI355X engine clocks settle only after ~300 encoder launches (~75 ms of
    sustained MFMA load); a fixed launch count warms a short run less than a
    long one, so the settle phase is bounded by time and reported in the line.
    """
    import torch
    t_end = time.perf_counter() + seconds
    n = 0
    while time.perf_counter() < t_end:
        for _ in range(20):
            fn()
        n += 20
        torch.cuda.synchronize()
    return n


def cpu_info() -> dict:
    """Host CPU model and the thread count the reference would use:
    std::thread::available_parallelism() is the affinity mask bounded by the
    cgroup CPU quota (bench_flash_attention_tiled.rs:247-249 uses it)."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    nproc = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, -(-int(q) // int(per)))
    except (OSError, ValueError):
        pass
    threads = min(nproc, quota) if quota else nproc
    return {"model": model, "nproc": nproc, "cgroup_cpus": quota, "threads": threads}


REPS = 9  # bench_flash_attention_tiled.rs:20


def time_both(a, b, reps: int = REPS):
    """bench_flash_attention_tiled.rs:109-134: best of `reps`, the two calls in
    alternating order so drift and background load bias both equally."""
    best_a = best_b = float("inf")
    for rep in range(reps):
        order = (a, b) if rep % 2 == 0 else (b, a)
        for f in order:
            t0 = time.perf_counter()
            f()
            dt = time.perf_counter() - t0
            if f is a:
                best_a = min(best_a, dt)
            else:
                best_b = min(best_b, dt)
    return best_a, best_b


def time_best(a, reps: int = REPS) -> float:
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        a()
        best = min(best, time.perf_counter() - t0)
    return best


def bench_encoder(wrs, W, ctx, steps, warmup, cfg=None, settle=True, graph=0):
    """One prefill launch over all windows per step, inputs resident in HBM:
    a time-bounded clock-settle phase, `warmup` untimed steps, then `steps`
    timed steps between two events on the launch stream. With `graph` > 0
    the steps are replays of a HIP graph of that many launches (checked
    against the eager result first), for launches shorter than the host's
    own call path."""
    import torch
    cfg = cfg or W.LARGE_ENCODER
    log(f"encoder: generating {cfg.name}")
    q, k, v = cfg.inputs()
    tdt = torch.bfloat16 if cfg.storage == "bf16" else torch.float16
    qd, kd, vd = (torch.from_numpy(x).to(tdt).cuda() for x in (q, k, v))
    B, T, dm = cfg.batch, cfg.t, cfg.d_model
    out = torch.empty((B, T, dm), dtype=torch.float32, device="cuda")
    lay = wrs.token_major(T, dm, 64)

    def launch():
        wrs.prefill(qd, kd, vd, out, batch=B, n_heads=cfg.n_heads, t_q=T, t_kv=T, d_head=64,
                    q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)

    step, per_step = launch, 1
    if graph > 0:
        launch()
        torch.cuda.synchronize()
        eager = out.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.use_torch_stream()
            for _ in range(graph):
                launch()
        ctx.use_torch_stream()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(out, eager):
            raise RuntimeError("graph replay of the encoder launches differs from eager")
        step, per_step = g.replay, graph
        steps, warmup = max(1, -(-steps // graph)), -(-warmup // graph)

    settled = 0
    if settle:
        log(f"encoder: settling clocks for {SETTLE_SECONDS} s")
        settled = settle_clocks(step)
    log(f"encoder: warmup {warmup}")
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"encoder: timing {steps * per_step} steps")
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / (steps * per_step)
    settled *= per_step
    tflops = cfg.flops() / (ms * 1e-3) / 1e12
    log(f"encoder: {cfg.name}: {ms:.4f} ms/step, {tflops:.1f} TFLOP/s "
        f"({tflops / PEAK_BF16_TFLOPS:.3f} of peak; settle {settled} launches)")
    return cfg, ms, tflops, (q, k, v), settled


def bench_one_window(wrs, W, ctx, steps, warmup):
    """The encoder attention of one 30 s window per call (the reference's
    encoder runs one window at a time): whisper-base (96 blocks of 128
    queries, fewer than half the CUs, which takes the key split) and large-v3
    (240 blocks, which takes key halves), each also under the 128-query
    schedule for comparison. The first leg settles the clocks; the launches
    are replayed from HIP graphs of 25, since one window's launch is shorter
    than the host's call path."""
    res = {}
    steps = max(steps, 100)
    for i, cfg in enumerate((W.BASE_ENCODER_1, W.LARGE_ENCODER_1)):
        _, ms, tf, _, _ = bench_encoder(wrs, W, ctx, steps, warmup, cfg=cfg, settle=i == 0,
                                        graph=25)
        ctx.set_schedule(prefill_queries=128)
        try:
            _, ms128, tf128, _, _ = bench_encoder(wrs, W, ctx, steps, warmup, cfg=cfg,
                                                  settle=False, graph=25)
        finally:
            ctx.set_schedule()
        res[cfg.name] = {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
                         "frac_mfma": round(tf / PEAK_BF16_TFLOPS, 4),
                         "wg128_us": round(ms128 * 1e3, 2), "wg128_TFLOPs": round(tf128, 1)}
    return res


def _replay_time_us(g, reps, launches_per_replay):
    import torch
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (reps * launches_per_replay)


# Launch shapes of the read-floor sweep: (threads per workgroup, 16-byte
# loads per lane), from 1875 down to 40 workgroups for 7.68 MB.
FLOOR_SHAPES = ((256, 1), (256, 4), (256, 8), (512, 2), (512, 4), (512, 8), (1024, 2),
                (1024, 4), (512, 24))


def bench_decode(wrs, W, ctx, reps, use_graph=True):
    """Cross-attention decode, one launch per layer over 32 resident layers,
    three utterances' caches rotated (737 MB > the 256 MB MALL), replayed
    from a HIP graph. Beside it, the practical floor of one decode-sized
    launch: a plain streaming read of the same 7.68 MB per launch, rotated
    the same way, at the fastest of several launch shapes
    (wrs_stream_read_shape)."""
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
    ctx.reserve(n_heads=cfg.n_heads, decode_rows=cfg.beams, decode_keys=cfg.n_audio)

    def all_layers():
        for u in range(U):
            for layer in range(cfg.n_layers):
                arenas[u].decode_cross(layer, qs[layer], outs[u, layer])

    all_layers()
    torch.cuda.synchronize()
    if not use_graph:  # eager launches (counter passes)
        for _ in range(reps):
            all_layers()
        torch.cuda.synchronize()
        for ar in arenas:
            ar.close()
        return cfg, float("nan"), float("nan"), None
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
    log(f"decode: timing {reps} graph replays of {U * cfg.n_layers} launches")
    us = _replay_time_us(g, reps, U * cfg.n_layers)
    gbs = cfg.bytes_per_layer() / (us * 1e-6) / 1e9
    # The floor: 7.68 MB per launch (two layers' K planes, contiguous), read
    # once by a plain streaming kernel, rotated like the decode, over launch
    # shapes from 40 to 1875 workgroups; the fastest shape is the floor.
    per = 2 * cfg.n_heads * cfg.n_audio * 64 * 2
    sink = torch.zeros(per // 4096 + 1, device="cuda")
    bases = [ar.plane_pointers()[2] for ar in arenas]

    def reads(threads, loads, nbytes):
        def fn():
            for base in bases:
                for pair in range(cfg.n_layers // 2):
                    ctx.check(ctx._lib.wrs_stream_read_shape(
                        ctx.handle, base + pair * per, nbytes, threads, loads, sink.data_ptr(),
                        sink.numel()), "wrs_stream_read_shape")
        return fn

    def replay_us(fn):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            ctx.use_torch_stream()
            fn()
        ctx.use_torch_stream()
        return _replay_time_us(gr, reps, U * cfg.n_layers // 2)

    shapes = {}
    for threads, loads in FLOOR_SHAPES:
        shapes[f"{threads}x{loads}"] = {
            "workgroups": -(-per // (16 * threads * loads)),
            "us_per_launch": round(replay_us(reads(threads, loads, per)), 3)}
    best = min(shapes, key=lambda k: shapes[k]["us_per_launch"])
    floor_us = shapes[best]["us_per_launch"]
    # and what any launch costs in these replays: one workgroup, one load
    tiny_us = replay_us(reads(256, 1, 16))
    floor = {"bytes_per_launch": per, "us_per_launch": floor_us,
             "GBps": round(per / (floor_us * 1e-6) / 1e9, 1),
             "best_shape": best + " (threads x 16-byte loads per lane)",
             "shapes": shapes, "one_workgroup_launch_us": round(tiny_us, 3)}
    log(f"decode: {us:.3f} us/launch ({gbs:.1f} GB/s); single-launch read floor "
        f"{floor_us:.3f} us ({floor['GBps']} GB/s, {best}); one-workgroup launch {tiny_us:.3f} us")
    for ar in arenas:
        ar.close()
    return cfg, us, gbs, floor


def bench_decode_self(wrs, W, ctx, reps, lengths=None, eager=False):
    """Causal self-attention decode, whisper-small shape (beam 5 slots, 12
    heads, max_ctx 448): one launch per layer over 12 layers, 8 arenas rotated
    so that the bytes read per round are larger than the 256 MB MALL, at each
    valid length L (the step's own row included)."""
    import torch
    lengths = lengths or W.SELF_DECODE_SWEEP
    base = W.SMALL_SELF_DECODE
    n_layers, U = 12, 8
    maxc = base.max_ctx
    log(f"decode self: building {U} x {n_layers}-layer self caches of {maxc} rows")
    full = W.SelfDecode(base.name, base.beams, base.n_heads, maxc)
    kvs = [full.kv(s) for s in range(base.beams)]
    kd = [(torch.from_numpy(k.astype(np.float32)).cuda(), torch.from_numpy(v.astype(np.float32)).cuda())
          for k, v in kvs]
    arenas = []
    for u in range(U):
        ar = wrs.KvArena(n_layers, base.beams, base.n_heads, maxc, 0, ctx=ctx)
        for s_ in range(base.beams):
            k, v = kd[s_]
            for layer in range(n_layers):
                ar.append(layer, s_, k, v)
            ar.advance(s_, maxc)
        arenas.append(ar)
    q = torch.from_numpy(base.q()).cuda()
    outs = torch.zeros((U, n_layers, base.beams, base.d_model), device="cuda")
    slots = list(range(base.beams))
    ctx.reserve(n_heads=base.n_heads, decode_rows=base.beams, decode_keys=maxc)

    def all_layers():
        for u in range(U):
            for layer in range(n_layers):
                arenas[u].decode_self(layer, slots, q, outs[u, layer])

    res = {}
    for L in lengths:
        for ar in arenas:
            for s_ in slots:
                # the rows stay in the planes: reset the length, then advance
                # it so that the step's own row sits at position L - 1
                ar.clear_slot(s_)
                ar.advance(s_, L - 1)
        all_layers()
        torch.cuda.synchronize()
        if eager:
            for _ in range(reps):
                all_layers()
            torch.cuda.synchronize()
            continue
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.use_torch_stream()
            all_layers()
        ctx.use_torch_stream()
        us = _replay_time_us(g, reps, U * n_layers)
        cfg = W.SelfDecode(base.name, base.beams, base.n_heads, L)
        gbs = cfg.bytes() / (us * 1e-6) / 1e9
        res[L] = {"us_per_launch": round(us, 3), "GBps": round(gbs, 1),
                  "bytes_per_launch": cfg.bytes(), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"decode self L={L}: {us:.3f} us/launch, {gbs:.1f} GB/s")
    if not eager:
        # The read floor at the headline length: the same bytes per launch,
        # contiguous, read once by a plain streaming kernel at its fastest
        # shape, rotated over the arenas and layers like the decode.
        L0 = base.ctx
        per = (W.SelfDecode(base.name, base.beams, base.n_heads, L0).bytes() + 15) // 16 * 16
        # the read windows stay inside each arena's self K planes
        k_plane_bytes = n_layers * base.beams * base.n_heads * maxc * 64 * 2
        n_fit = k_plane_bytes // per
        assert n_fit >= 1
        sink = torch.zeros(per // 4096 + 1, device="cuda")
        bases = [ar.plane_pointers()[0] for ar in arenas]

        def reads(threads, loads):
            def fn():
                for bp in bases:
                    for layer in range(n_layers):
                        ctx.check(ctx._lib.wrs_stream_read_shape(
                            ctx.handle, bp + (layer % n_fit) * per, per, threads, loads,
                            sink.data_ptr(), sink.numel()), "wrs_stream_read_shape")
            return fn

        best = None
        for threads, loads in ((256, 1), (256, 4), (512, 2), (512, 4)):
            fn = reads(threads, loads)
            fn()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                ctx.use_torch_stream()
                fn()
            ctx.use_torch_stream()
            t = _replay_time_us(gr, reps, U * n_layers)
            if best is None or t < best[0]:
                best = (t, f"{threads}x{loads}")
        res["floor"] = {"length": L0, "bytes_per_launch": per, "us_per_launch": round(best[0], 3),
                        "best_shape": best[1] + " (threads x 16-byte loads per lane)"}
        log(f"decode self: read floor at L={L0}: {best[0]:.3f} us ({best[1]})")
    for ar in arenas:
        ar.close()
    return res


def bench_capture(wrs, W, ctx, reps, use_graph=True, one_pass=True):
    """DTW alignment pass: one capture call per preset layer, inputs resident.

    one_pass: each layer's capture reads the row statistics that the layer's
    cross-attention over the same rows left (decoder.rs:698-721's order; that
    attention call, made once before timing, is the decoder's own work and not
    timed here): one launch per call. Otherwise the two-pass capture of the
    reference-shaped entry point, which computes its own statistics."""
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
    lse = {}
    rows_us = float("nan")
    if one_pass:
        att = torch.zeros((cfg.n_tokens, cfg.d_model), device="cuda")
        for layer in layers:
            lse[layer] = torch.zeros(2 * cfg.n_heads * cfg.n_tokens, device="cuda")
            ar.prefill_cross(layer, qs[layer], att, lse=lse[layer])
        torch.cuda.synchronize()
        if use_graph:
            # the decoder's own cross-attention of the same rows (its output and
            # the statistics), timed on its own: decoder.rs:698-708 per layer
            ga = torch.cuda.CUDAGraph()
            with torch.cuda.graph(ga):
                ctx.use_torch_stream()
                for layer in layers:
                    ar.prefill_cross(layer, qs[layer], att, lse=lse[layer])
            ctx.use_torch_stream()
            for _ in range(3):
                ga.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                ga.replay()
            e1.record()
            torch.cuda.synchronize()
            rows_us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
            log(f"capture: the layers' cross-attention of the {cfg.n_tokens} rows with "
                f"statistics: {rows_us:.2f} us per layer")

    def all_layers():
        for layer in layers:
            ar.capture_cross_heads(layer, qs[layer], cfg.pairs(layer), n_sel, 0, out,
                                   lse=lse.get(layer))

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
    log(f"capture ({'one pass' if one_pass else 'two passes'}): timing {reps} graph replays "
        f"of {len(layers)} calls")
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / (reps * len(layers))
    gbs = cfg.bytes_per_pair() / (us * 1e-6) / 1e9  # one pair per preset layer
    ar.close()
    bench_capture.rows_us = rows_us
    return cfg, us, gbs


def bench_linear(wrs, cfg, ctx, reps, settle=True):
    """One fused QKV projection per step, inputs resident; bf16 rows out."""
    import torch
    x = torch.from_numpy(cfg.x()).cuda()
    if cfg.x_storage == "f16":
        x = x.half()
    w = torch.from_numpy(cfg.w()).cuda()
    b = torch.from_numpy(cfg.bias()).cuda()
    out = torch.empty((cfg.n_tokens, cfg.n_out), dtype=torch.bfloat16, device="cuda")
    if settle:
        settle_clocks(lambda: wrs.linear(x, w, b, out, ctx=ctx), 0.5)
    else:
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


def bench_weight_stream(wrs, W, ctx, reps, eager=False):
    """One decoder step's projections for 5 beams, replayed from a HIP graph:
    every launch streams its f16 weights once (the decode-sized linear path).
    `eager` runs `reps` plain steps and returns (counter passes)."""
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

    if eager:  # exactly `reps` steps, nothing else (counter passes)
        for _ in range(reps):
            step()
        torch.cuda.synchronize()
        return cfg, len(calls)
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
    one write. LayerNorm's 184 MB per call would fit the 256 MB MALL, so its
    calls rotate over four input/output pairs (737 MB); GELU's 491 MB working
    set does not fit."""
    import torch
    gen = torch.Generator(device="cuda").manual_seed(0x5EED)
    T, d = 24000, 1280
    n_rot = 4
    xs = [torch.randn((T, d), generator=gen, device="cuda") for _ in range(n_rot)]
    g = torch.randn(d, generator=gen, device="cuda")
    b = torch.randn(d, generator=gen, device="cuda")
    ys = [torch.empty((T, d), dtype=torch.bfloat16, device="cuda") for _ in range(n_rot)]
    h = torch.randn((T, 4 * d), generator=gen, device="cuda")
    turn = [0]

    def layer_norm():
        i = turn[0] % n_rot
        turn[0] += 1
        wrs.layer_norm(xs[i], g, b, 1e-5, ys[i], ctx=ctx)

    res = {}
    for name, fn, nbytes in (("layer_norm", layer_norm, T * d * (4 + 2)),
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


def device_call_ms(ctx, run, out, reps: int, per_graph: int = 10) -> float:
    """Mean time of one launch of `run` (which writes `out`), in ms, from HIP
    graph replays of `per_graph` launches checked against the eager result:
    timed from the host, launches shorter than its call path would time the
    host instead."""
    import torch
    run()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.use_torch_stream()
        for _ in range(per_graph):
            run()
    ctx.use_torch_stream()
    out.zero_()
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(out, eager):
        raise RuntimeError("graph replay of the launch differs from eager")
    return _replay_time_us(g, max(1, reps), per_graph) / 1e3


def host_call_ms(fn, reps: int) -> dict:
    """Per-call wall times of a synchronous host-slice call, in ms: the
    median (the figure reported; single calls through pageable host memory
    now and then stall for tens of milliseconds), the mean and the best."""
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return {"median": float(np.median(ts)), "mean": float(np.mean(ts)), "best": min(ts)}


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
    host = host_call_ms(lambda: wrs.flash_attention_2(q, k, v, T, T, H, dm, False, out, ctx=ctx),
                        reps)
    host_ms = host["median"]
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    od = torch.empty_like(qd)
    lay = wrs.token_major(T, dm, 64)
    run = lambda: wrs.prefill(qd, kd, vd, od, batch=1, n_heads=H, t_q=T, t_kv=T, d_head=64,
                              q_layout=lay, kv_layout=lay, out_layout=lay, ctx=ctx)
    for _ in range(20):
        run()
    torch.cuda.synchronize()
    dev_ms = device_call_ms(ctx, run, od, reps)
    gflop = cfg.flops() / 1e9
    return {"workload": cfg.name, "unit": "GFLOP/s",
            "host_slice_ms": round(host_ms, 3), "host_slice_value": round(gflop / host_ms * 1e3, 1),
            "host_slice_mean_ms": round(host["mean"], 3),
            "host_slice_best_ms": round(host["best"], 3),
            "device_resident_ms": round(dev_ms, 4),
            "device_resident_value": round(gflop / dev_ms * 1e3, 1),
            "pcie_bytes_per_call": 4 * q.nbytes}


# (t_q, t_kv) of the reference's attention microbenchmark, 6 heads of 64
# (crates/tensor/tests/bench_flash_attention_tiled.rs:19-25): an encoder row of
# 1500 frames, a 64-row cross-attention call, and a shape whose score matrix
# outgrows the last-level cache.
REFERENCE_SHAPES = ((1500, 1500), (64, 1500), (4096, 4096))


def _reference_shape_inputs(t_q, t_kv, n_heads=6):
    """f32 Q, K, V uniform in [-1, 1), seeded per shape (the microbenchmark's
    value range; its own generator is xorshift32)."""
    rng = np.random.default_rng(0x5EED0000 + 7919 * t_q + t_kv)
    dm = 64 * n_heads
    return tuple(rng.uniform(-1.0, 1.0, size=(t, dm)).astype(np.float32)
                 for t in (t_q, t_kv, t_kv))


def bench_reference_shapes(wrs, ctx, reps=20):
    """flash_attention_2 at the reference microbenchmark's shapes, f32, no mask:
    the host-slice drop-in (PCIe both ways, synchronous; median per call of
    `reps`) and the same call on device-resident tensors (the f32 prefill
    kernel), per shape."""
    import torch
    res = {}
    H = 6
    for t_q, t_kv in REFERENCE_SHAPES:
        q, k, v = _reference_shape_inputs(t_q, t_kv, H)
        dm = q.shape[1]
        out = np.empty_like(q)
        for _ in range(3):
            wrs.flash_attention_2(q, k, v, t_q, t_kv, H, dm, False, out, ctx=ctx)
        host = host_call_ms(
            lambda: wrs.flash_attention_2(q, k, v, t_q, t_kv, H, dm, False, out, ctx=ctx), reps)
        host_ms = host["median"]
        qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
        od = torch.empty_like(qd)
        lq, lkv = wrs.token_major(t_q, dm, 64), wrs.token_major(t_kv, dm, 64)
        run = lambda: wrs.prefill(qd, kd, vd, od, batch=1, n_heads=H, t_q=t_q, t_kv=t_kv,
                                  d_head=64, q_layout=lq, kv_layout=lkv, out_layout=lq, ctx=ctx)
        for _ in range(20):
            run()
        torch.cuda.synchronize()
        dev_ms = device_call_ms(ctx, run, od, reps)
        gflop = 4.0 * H * t_q * t_kv * 64 / 1e9
        res[f"{t_q}x{t_kv}"] = {
            "host_slice_ms": round(host_ms, 4),
            "host_slice_GFLOPs": round(gflop / host_ms * 1e3, 1),
            "host_slice_mean_ms": round(host["mean"], 4),
            "host_slice_best_ms": round(host["best"], 4),
            "device_resident_ms": round(dev_ms, 4),
            "device_resident_GFLOPs": round(gflop / dev_ms * 1e3, 1),
            "pcie_bytes_per_call": q.nbytes + k.nbytes + v.nbytes + out.nbytes}
        log(f"reference shape ({t_q}, {t_kv}) x {H} heads: host slices {host_ms:.3f} ms, "
            f"device-resident {dev_ms * 1e3:.1f} us ({gflop / dev_ms:.1f} TFLOP/s)")
        del qd, kd, vd, od
    return res


def cpu_baseline_reference_shapes(info):
    """The oracle's tiled flash_attention_2 at the same shapes and inputs, best
    of 9 on available_parallelism() threads (best of 3 at (4096, 4096))."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    n = info["threads"]
    res = {}
    for t_q, t_kv in REFERENCE_SHAPES:
        q, k, v = (np.ascontiguousarray(x.reshape(-1)) for x in _reference_shape_inputs(t_q, t_kv))
        dm = 384
        out = np.zeros_like(q)
        fn = lambda: orc.flash_attention_2(q, k, v, t_q, t_kv, 6, dm, False, out, n_threads=n)
        fn()
        t = time_best(fn, reps=3 if t_q * t_kv > 4_000_000 else REPS)
        gflop = 4.0 * 6 * t_q * t_kv * 64 / 1e9
        res[f"{t_q}x{t_kv}"] = {"ms": round(t * 1e3, 2), "GFLOPs": round(gflop / t, 1),
                                "cores": n, "kind": "port"}
    return res


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


def read_bandwidth(ctx):
    """Read-only streaming rate over 1 GiB (wrs_stream_read_shape, 256 threads x
    eight 16-byte loads per lane): the ceiling of a pure read stream, beside the
    copy's 1:1 read/write mix."""
    import torch
    nbytes = 1 << 30
    a = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(nbytes // (16 * 256 * 8) + 1, device="cuda")

    def run():
        ctx.check(ctx._lib.wrs_stream_read_shape(ctx.handle, a.data_ptr(), nbytes, 256, 8,
                                                 sink.data_ptr(), sink.numel()),
                  "wrs_stream_read_shape")

    run()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(10):
        run()
    e.record()
    torch.cuda.synchronize()
    return nbytes / (s.elapsed_time(e) / 10 * 1e-3) / 1e9


CALIB_BYTES = 256 << 20  # one plain device copy of this many bytes per profiled run


def calibration_copy():
    """A plain copy of known size: the reference point for FETCH_SIZE/WRITE_SIZE."""
    import torch
    a = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


# kernel-name patterns of each leg in the counter passes (demangled names)
TRAFFIC_LEGS = {
    # demangled (fa2_prefill_d64<__bf16, ...>) or mangled (fa2_prefill_d64IDF16b...);
    # rocprofv3's demangler can also print the __bf16 argument as "bool _Accum"
    "encoder": (r"fa2_prefill_d64(?:<\s*|I)(?:__bf16|bf16|DF16b|bool _Accum)", None),
    "encoder_base": (r"fa2_prefill_d64(?:<\s*|I)(?:_Float16|half|DF16_)", None),
    "decode": (r"decode_f16<\s*5\s*,", None),
    "decode_self": (r"decode_f16<\s*1\s*,", None),
    # capture_cross_f16<2> is the one-pass kernel, <0> and <1> the two passes
    "capture": (r"capture_cross_f16(?:<\s*|ILi)2", None),
    "capture_two_pass": (r"capture_cross_f16(?:<\s*|ILi)[01]", None),
    "linear": (r"linear_f16w", None),
    "stream": (r"gemv_f16w", "per_step"),
}


def measure_traffic(extra: list[str]):
    """HBM bytes per call of every leg's kernel(s).

    Two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch)
    over `bench.py --only traffic`, which runs every leg eagerly a few times;
    each counter is scaled by what it reads for the plain device copy of
    CALIB_BYTES in the same run. Returns {leg: {...}} (legs whose kernels are
    missing are left out), or None when rocprofv3 is unavailable or a pass
    fails.
    """
    import re
    if shutil.which("rocprofv3") is None:
        return None
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory(dir="/tmp") as d:
            cmd = ["timeout", "-s", "KILL", "300", "rocprofv3", "--pmc", counter, "-d", d, "-o",
                   "t", "--", sys.executable, str(Path(__file__).resolve()), "--only",
                   "traffic"] + extra
            env = dict(os.environ, TMPDIR="/tmp")
            log(f"traffic: {counter} pass")
            r = subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, env=env,
                               cwd="/tmp")
            dbs = list(Path(d).rglob("*_results.db"))
            if r.returncode != 0 or not dbs:
                log(f"traffic: {counter} pass failed (rc={r.returncode})")
                return None
            db = sqlite3.connect(str(dbs[0]))
            rows = db.execute("select kernel_name, avg(value), max(value), sum(value), count(*) "
                              "from counters_collection where counter_name = ? "
                              "group by kernel_name", (counter,)).fetchall()
            db.close()
            # the calibration copy is the largest dispatch of its kernel: other,
            # smaller copies (input set-up) can share the kernel's name
            copy = [vmax for n, _, vmax, _, _ in rows
                    if "copy" in n.lower() or "elementwise" in n.lower()]
            if not copy or max(copy) <= 0:
                log(f"traffic: {counter}: no calibration copy in the profile")
                return None
            factor = CALIB_BYTES / (max(copy) * 1024.0)
            if counter == "FETCH_SIZE":
                log("traffic: kernels profiled: " +
                    "; ".join(f"{n[:90]} x{c}" for n, _, _, _, c in rows))
            for leg, (pat, mode) in TRAFFIC_LEGS.items():
                hit = [(n, av, tot, cnt) for n, av, _, tot, cnt in rows if re.search(pat, n)]
                if not hit:
                    continue
                if mode == "per_step":
                    steps = TRAFFIC_STREAM_STEPS
                    kib = sum(t for _, _, t, _ in hit) / steps
                else:
                    # one call = one dispatch of each matching kernel (the
                    # capture runs as two passes)
                    kib = sum(av for _, av, _, _ in hit)
                res.setdefault(leg, {})[counter] = kib * 1024.0 * factor
                res[leg][counter + "_factor"] = round(factor, 4)
                log(f"traffic: {leg} {counter} = {kib:.1f} KiB per call over "
                    f"{len(hit)} kernel(s); factor {factor:.4f}")
    return {leg: v for leg, v in res.items() if "FETCH_SIZE" in v and "WRITE_SIZE" in v}


TRAFFIC_STREAM_STEPS = 3


def run_traffic_legs(wrs, W, ctx):
    """Every leg a few times, eagerly, then the calibration copy: the program
    the counter passes profile."""
    bench_encoder(wrs, W, ctx, 3, 1, settle=False)
    bench_encoder(wrs, W, ctx, 3, 1, cfg=W.BASE_ENCODER, settle=False)
    bench_decode(wrs, W, ctx, 3, use_graph=False)
    bench_decode_self(wrs, W, ctx, 3, lengths=(W.SMALL_SELF_DECODE.ctx,), eager=True)
    bench_capture(wrs, W, ctx, 3, use_graph=False)
    bench_capture(wrs, W, ctx, 3, use_graph=False, one_pass=False)
    bench_linear(wrs, W.LARGE_QKV_F16, ctx, 3, settle=False)
    bench_weight_stream(wrs, W, ctx, TRAFFIC_STREAM_STEPS, eager=True)
    calibration_copy()


def cpu_baseline_encoder(cfg, qkv, info):
    """The oracle's tiled flash_attention_2 on one window, timed by the
    reference's method (bench_flash_attention_tiled.rs:109-134, :240-249):
    one warm call each, then best of 9 alternating with the materialized
    baseline, on available_parallelism() threads."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    q, k, v = (np.ascontiguousarray(x[0].reshape(-1)) for x in qkv)
    out = np.zeros_like(q)
    mat = np.zeros_like(q)
    T, H, dm = cfg.t, cfg.n_heads, cfg.d_model
    n = info["threads"]
    tiled = lambda: orc.flash_attention_2(q, k, v, T, T, H, dm, False, out, n_threads=n)
    base = lambda: orc.materialized_attention(q, k, v, T, T, H, dm, mat, n_threads=n)
    tiled()
    base()
    t_tiled, t_mat = time_both(tiled, base)
    flops = 4.0 * H * T * T * 64
    return {"value": round(flops / t_tiled / 1e12, 4), "unit": "TFLOP/s", "cores": n,
            "kind": "port",
            "materialized_value": round(flops / t_mat / 1e12, 4),
            "cpu": info["model"], "nproc": info["nproc"], "cgroup_cpus": info["cgroup_cpus"],
            "sample": f"1 of {cfg.batch} windows ({H} heads x {T} x {T}); the oracle's tiled "
                      f"flash_attention_2 best of {REPS} alternating with its materialized "
                      f"baseline (bench_flash_attention_tiled.rs method), "
                      f"{t_tiled * 1e3:.1f} ms vs {t_mat * 1e3:.1f} ms"}


def cpu_baseline_decode(cfg, info):
    """One layer's cross-attention decode: single_token_mha_d64 for each beam in
    turn over f32 K/V (the reference's serial per-slot loop,
    decoder.rs:689-724), one thread, best of 9 after a warm call."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    kk, vv = cfg.kv(0)
    k, v = np.ascontiguousarray(kk.ravel()), np.ascontiguousarray(vv.ravel())
    q = cfg.q(0)
    out = np.zeros(cfg.d_model, np.float32)

    def layer():
        for b in range(cfg.beams):
            orc.single_token_mha_d64(np.ascontiguousarray(q[b]), k, v, cfg.n_audio, cfg.n_heads,
                                     cfg.d_model, out)

    layer()
    best = time_best(layer)
    return {"value": round(cfg.bytes_per_layer() / best / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port", "cpu": info["model"],
            "sample": f"1 layer, {cfg.beams} beams read serially from f32 K/V, best of {REPS}, "
                      f"{best * 1e3:.3f} ms"}


def cpu_baseline_decode_self(W, L, info):
    """One layer's self-attention decode at valid length L: the reference's
    per-slot loop (decoder.rs:617-647) calling single_token_mha_d64 over each
    slot's f32 cache of L rows (decoder.rs:852-855), one thread."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    cfg = W.SelfDecode(W.SMALL_SELF_DECODE.name, W.SMALL_SELF_DECODE.beams,
                       W.SMALL_SELF_DECODE.n_heads, L)
    kvs = [tuple(np.ascontiguousarray(x.ravel()) for x in cfg.kv(s)) for s in range(cfg.beams)]
    q = cfg.q()
    out = np.zeros(cfg.d_model, np.float32)

    def layer():
        for s_ in range(cfg.beams):
            k, v = kvs[s_]
            orc.single_token_mha_d64(np.ascontiguousarray(q[s_]), k, v, L, cfg.n_heads,
                                     cfg.d_model, out)

    layer()
    best = time_best(layer)
    return {"value": round(cfg.bytes() / best / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port", "cpu": info["model"],
            "sample": f"1 layer, {cfg.beams} slots x {L} rows read serially from f32 K/V, best "
                      f"of {REPS}, {best * 1e6:.1f} us"}


def cpu_baseline_capture(cfg):
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    layer = cfg.layers()[0]
    q = np.ascontiguousarray(cfg.q(layer).ravel())
    k = np.ascontiguousarray(cfg.k(layer).ravel())
    sel = cfg.pairs(layer)
    out = np.zeros(cfg.n_tokens * len(cfg.heads) * cfg.n_audio, np.float32)
    run = lambda: orc.capture_cross_attention_heads(q, k, cfg.n_tokens, cfg.n_audio, cfg.n_heads,
                                                    cfg.d_model, sel, len(cfg.heads), 0, out)
    run()
    best = time_best(run)
    return {"value": round(cfg.bytes_per_pair() / best / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"1 layer's pair ({cfg.n_tokens} tokens x {cfg.n_audio} frames), best of "
                      f"{REPS}, {best * 1e3:.2f} ms"}


def cpu_baseline_linear(cfg, threads):
    """The oracle's f16_linear on one 1500-frame window of the batch."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    n = 1500
    x = np.ascontiguousarray(cfg.x()[:n].astype(np.float32).ravel())
    w = np.ascontiguousarray(cfg.w())
    b = cfg.bias()
    out = np.zeros(n * cfg.n_out, np.float32)
    run = lambda: orc.f16_linear(w, cfg.n_out, cfg.n_in, x, b, n, out, n_threads=threads)
    run()
    best = time_best(run)
    flops = 2.0 * n * cfg.n_in * cfg.n_out
    return {"value": round(flops / best / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"1 window of 16 ({n} x {cfg.n_in} x {cfg.n_out}), best of {REPS}, "
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
    def run():
        for w in ws:
            r, c = w.shape
            orc.f16_linear(w, r, c, xs[c], None, cfg.beams, outs[r], n_threads=threads)

    run()
    best = time_best(run)
    nbytes = sum(r * c * 2 for r, c in mats)
    return {"value": round(nbytes / best / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"one layer's 8 projections ({nbytes / 1e6:.1f} MB of f16 weights, "
                      f"{cfg.beams} rows), best of {REPS}, {best * 1e3:.2f} ms"}


def _roof(achieved, peak, unit, bound, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # untimed steps after the time-bounded clock-settle phase
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--decode-reps", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--eager", action="store_true",
                    help="with --only decode/decode_self/capture: plain launches, no graph")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 HBM-traffic passes")
    ap.add_argument("--capture-reps", type=int, default=100)
    ap.add_argument("--linear-reps", type=int, default=50)
    ap.add_argument("--linear-f16-only", action="store_true",
                    help="with --only linear: the f16-activation projection only")
    ap.add_argument("--stream-reps", type=int, default=20)
    ap.add_argument("--rows-reps", type=int, default=50)
    ap.add_argument("--only", choices=["encoder", "encoder_base", "decode", "decode_self",
                                       "capture", "linear", "stream", "rows", "host_slice",
                                       "reference_shapes", "one_window", "traffic"],
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

    if args.only == "traffic":
        run_traffic_legs(wrs, W, ctx)
        return
    if args.only == "one_window":
        log(f"one window: {bench_one_window(wrs, W, ctx, args.steps, max(args.warmup, 100))}")
        return
    if args.only in ("encoder", "encoder_base"):
        cfg = W.LARGE_ENCODER if args.only == "encoder" else W.BASE_ENCODER
        _, ms, tflops, _, n = bench_encoder(wrs, W, ctx, args.steps, args.warmup, cfg=cfg,
                                            graph=0 if args.only == "encoder" else 25)
        calibration_copy()
        log(f"{args.only} only: {ms:.4f} ms/step, {tflops:.1f} TFLOP/s (settle {n} launches)")
        return
    if args.only == "decode":
        _, us, gbs, floor = bench_decode(wrs, W, ctx, args.decode_reps, use_graph=not args.eager)
        calibration_copy()
        log(f"decode only: {us:.3f} us/launch, {gbs:.1f} GB/s; floor {floor}")
        return
    if args.only == "decode_self":
        res = bench_decode_self(wrs, W, ctx, args.decode_reps, eager=args.eager)
        calibration_copy()
        log(f"decode self only: {res}")
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
        log(f"rows only: device copy {copy_bandwidth():.1f} GB/s, read stream "
            f"{read_bandwidth(ctx):.1f} GB/s")
        calibration_copy()
        return
    if args.only == "stream":
        _, sms, sgbs, vms, vgbs, snorms = bench_weight_stream(wrs, W, ctx, args.stream_reps)
        calibration_copy()
        log(f"stream only: step {sms:.3f} ms, {sgbs:.1f} GB/s; vocabulary {vms * 1e3:.1f} us, "
            f"{vgbs:.1f} GB/s")
        return
    if args.only == "reference_shapes":
        bench_reference_shapes(wrs, ctx)
        return
    if args.only == "host_slice":
        hs = bench_host_slice(wrs, W, ctx, reps=100)
        log(f"host_slice only: host slices {hs['host_slice_ms']:.3f} ms/call, "
            f"device-resident {hs['device_resident_ms'] * 1e3:.1f} us/call "
            f"({hs['device_resident_value'] / 1e3:.1f} TFLOP/s)")
        return
    if args.only == "capture":
        _, cus, cgbs = bench_capture(wrs, W, ctx, args.capture_reps, use_graph=not args.eager)
        _, cus2, cgbs2 = bench_capture(wrs, W, ctx, args.capture_reps, use_graph=not args.eager,
                                       one_pass=False)
        calibration_copy()
        log(f"capture only: one pass {cus:.3f} us/call, {cgbs:.1f} GB/s; two passes "
            f"{cus2:.3f} us/call, {cgbs2:.1f} GB/s")
        return

    cfg, ms, tflops, qkv, settled = bench_encoder(wrs, W, ctx, args.steps, args.warmup)
    # whisper-base x4 (~30 us a launch) from graph replays, like one window:
    # its launch is about as long as the host's call path.
    bcfg, bms, btflops, bqkv, bsettled = bench_encoder(wrs, W, ctx, args.steps, args.warmup,
                                                       cfg=W.BASE_ENCODER, graph=25)
    one_window = bench_one_window(wrs, W, ctx, args.steps, max(args.warmup, 100))
    dcfg, us, gbs, floor = bench_decode(wrs, W, ctx, args.decode_reps)
    sweep = bench_decode_self(wrs, W, ctx, args.decode_reps)
    ccfg, cus, cgbs = bench_capture(wrs, W, ctx, args.capture_reps)
    cross_rows_us = bench_capture.rows_us
    _, cus2, cgbs2 = bench_capture(wrs, W, ctx, args.capture_reps, one_pass=False)
    lcfg = W.LARGE_QKV_F16
    lms, ltf = bench_linear(wrs, lcfg, ctx, args.linear_reps)
    lms32, ltf32 = bench_linear(wrs, W.LARGE_QKV_F32, ctx, args.linear_reps)
    scfg, sms, sgbs, vms, vgbs, snorms = bench_weight_stream(wrs, W, ctx, args.stream_reps)
    rows = bench_rows(wrs, ctx, args.rows_reps)
    log("host-slice drop-in: whisper-tiny encoder, f32 host slices")
    host_slice = bench_host_slice(wrs, W, ctx)
    log("reference microbenchmark shapes, f32")
    ref_shapes = bench_reference_shapes(wrs, ctx)
    copy_gbs = copy_bandwidth()
    read_gbs = read_bandwidth(ctx)

    traffic = None
    if not args.no_traffic:
        log("traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE passes")
        traffic = measure_traffic([])

    def traffic_bytes(leg):
        if not traffic or leg not in traffic:
            return None
        return round(traffic[leg]["FETCH_SIZE"] + traffic[leg]["WRITE_SIZE"])

    info = cpu_info()
    n = info["threads"]
    cpu = {}
    if not args.no_cpu:
        log(f"cpu baseline: oracle encoder windows on {n} threads ({info['model']})")
        cpu["encoder"] = cpu_baseline_encoder(cfg, qkv, info)
        cpu["encoder_base"] = cpu_baseline_encoder(bcfg, bqkv, info)
        log("cpu baseline: oracle decode layers, 1 thread")
        cpu["decode"] = cpu_baseline_decode(dcfg, info)
        cpu["decode_self"] = cpu_baseline_decode_self(W, W.SMALL_SELF_DECODE.ctx, info)
        log("cpu baseline: oracle capture of one layer, 1 thread")
        cpu["capture"] = cpu_baseline_capture(ccfg)
        log(f"cpu baseline: oracle f16_linear, one window, {n} threads")
        cpu["linear"] = cpu_baseline_linear(lcfg, n)
        log(f"cpu baseline: oracle f16_linear, one decoder layer's projections, {n} threads")
        cpu["stream"] = cpu_baseline_stream(scfg, n)
        log(f"cpu baseline: oracle flash_attention_2 at the reference shapes, {n} threads")
        cpu["reference_shapes"] = cpu_baseline_reference_shapes(info)

    L0 = W.SMALL_SELF_DECODE.ctx
    self_floor = sweep.pop("floor", None)
    self_ref = sweep[L0]
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
                   "frames": cfg.t, "d_head": 64, "flops_per_step": cfg.flops(),
                   "clock_settle": {"seconds": SETTLE_SECONDS, "launches": settled,
                                    "then_warmup_steps": args.warmup}},
        "roofline": _roof(tflops, PEAK_BF16_TFLOPS, "TFLOP/s", "mfma", traffic_bytes("encoder")),
        "cpu_baseline": cpu.get("encoder"),
        "encoder_base": {
            "workload": bcfg.name, "value": round(btflops, 2), "unit": "TFLOP/s",
            "ms_per_step": round(bms, 4), "flops_per_step": bcfg.flops(), "dtype": "f16",
            "clock_settle_launches": bsettled,
            "roofline": _roof(btflops, PEAK_BF16_TFLOPS, "TFLOP/s", "mfma",
                              traffic_bytes("encoder_base")),
            "cpu_baseline": cpu.get("encoder_base"),
        },
        "encoder_one_window": one_window,
        "decode_cross": {
            "workload": dcfg.name, "value": round(gbs, 1), "unit": "GB/s",
            "us_per_launch": round(us, 3), "launches_per_step": dcfg.n_layers,
            "bytes_per_launch": dcfg.bytes_per_layer(), "dtype": "f16",
            "roofline": _roof(gbs, PEAK_HBM_GBS, "GB/s", "hbm", traffic_bytes("decode")),
            "single_launch_read_floor": floor,
            "frac_of_read_floor": round(floor["us_per_launch"] / us, 4) if floor else None,
            "cpu_baseline": cpu.get("decode"),
        },
        "decode_self": {
            "workload": W.SMALL_SELF_DECODE.name + f", valid length {L0} of "
                                                   f"{W.SMALL_SELF_DECODE.max_ctx}",
            "value": self_ref["GBps"], "unit": "GB/s", "us_per_launch": self_ref["us_per_launch"],
            "launches_per_step": 12, "bytes_per_launch": self_ref["bytes_per_launch"],
            "dtype": "f16",
            "roofline": _roof(self_ref["GBps"], PEAK_HBM_GBS, "GB/s", "hbm",
                              traffic_bytes("decode_self")),
            "sweep": {str(L): v for L, v in sweep.items()},
            "single_launch_read_floor": self_floor,
            "frac_of_read_floor": (round(self_floor["us_per_launch"] / self_ref["us_per_launch"], 4)
                                   if self_floor else None),
            "cpu_baseline": cpu.get("decode_self"),
        },
        "capture": {
            "workload": ccfg.name, "value": round(cgbs, 1), "unit": "GB/s",
            "us_per_launch": round(cus, 3), "launches_per_step": len(ccfg.layers()),
            "bytes_per_launch": ccfg.bytes_per_pair(), "dtype": "f32",
            "roofline": _roof(cgbs, PEAK_HBM_GBS, "GB/s", "hbm", traffic_bytes("capture")),
            "mode": "one launch per call, on the row statistics of the layer's cross-attention",
            "cross_attention_rows_us_per_layer": round(cross_rows_us, 2),
            "two_pass": {"us_per_call": round(cus2, 3), "GBps": round(cgbs2, 1),
                         "roofline": _roof(cgbs2, PEAK_HBM_GBS, "GB/s", "hbm",
                                           traffic_bytes("capture_two_pass"))},
            "cpu_baseline": cpu.get("capture"),
        },
        "projection": {
            "workload": lcfg.name, "value": round(ltf, 2), "unit": "TFLOP/s",
            "ms_per_launch": round(lms, 4), "flops_per_launch": lcfg.flops(), "dtype": "f16",
            "roofline": _roof(ltf, PEAK_BF16_TFLOPS, "TFLOP/s", "mfma", traffic_bytes("linear")),
            "f32_exact": {"workload": W.LARGE_QKV_F32.name, "value": round(ltf32, 2),
                          "unit": "TFLOP/s", "ms_per_launch": round(lms32, 4)},
            "cpu_baseline": cpu.get("linear"),
        },
        "decoder_weight_stream": {
            "workload": scfg.name, "value": round(sgbs, 1), "unit": "GB/s",
            "ms_per_step": round(sms, 4), "launches_per_step": scfg.launches(),
            "weight_bytes_per_step": scfg.weight_bytes(), "dtype": "f16",
            "roofline": _roof(sgbs, PEAK_HBM_GBS, "GB/s", "hbm", traffic_bytes("stream")),
            "vocabulary_projection": {"us": round(vms * 1e3, 2), "GBps": round(vgbs, 1),
                                      "frac_hbm": round(vgbs / PEAK_HBM_GBS, 4)},
            "with_layer_norms_and_gelu": snorms,
            "cpu_baseline": cpu.get("stream"),
        },
        "row_kernels": rows,
        "host_slice": host_slice,
        "reference_shapes": {
            "workload": "flash_attention_2 at the reference microbenchmark's (t_q, t_kv), "
                        "6 heads x 64, f32, no mask",
            "gpu": ref_shapes, "cpu_baseline": cpu.get("reference_shapes")},
        "device": {"name": props.name, "cu": props.multi_processor_count,
                   "copy_GBps": round(copy_gbs, 1), "read_GBps": round(read_gbs, 1)},
        "host": info,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
