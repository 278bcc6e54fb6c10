"""Concurrency contract of the C ABI (include/wrs_attn.h: one context per
thread, independent contexts may run concurrently), as the reference runs
attention from OS threads in whisper_full_parallel
(crates/ffi/src/lib.rs:1378-1440, std::thread::scope).

Four host threads each own a context (and its stream) and, at the same time,
run synchronous host-slice calls (flash_attention_2 on f32 host slices) and
asynchronous device-resident calls (an f16 encoder prefill and a beam-5
cross-attention decode over their own arena). Threads 0 and 2 take the shapes
whose work is merged through the context's scratch: the 64-query host slice
over 1500 keys (each block's tiles over twelve workgroups) and one
whisper-base window (each 128-query block over two workgroups). Every result is compared with
the oracle's, computed beforehand on the same inputs; a thread stops at its
first failure and the test reports it. ctypes releases the GIL for the
duration of each library call, so the calls do overlap in the library.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

from gpu_util import dev, host, note

pytestmark = pytest.mark.gpu

N_THREADS = 4
ROUNDS = 6


def _oracle_fa2(orc, q, k, v, t_q, t_kv, h, dm, causal=False):
    out = np.zeros(t_q * dm, np.float32)
    orc.flash_attention_2(np.ascontiguousarray(q.ravel()), np.ascontiguousarray(k.ravel()),
                          np.ascontiguousarray(v.ravel()), t_q, t_kv, h, dm, causal, out)
    return out.reshape(t_q, dm)


def _case(orc, W, i):
    """Inputs and oracle results of thread i (distinct seeds per thread)."""
    c = {}
    # host slice, f32: (100, 137) keys, 3 heads of 64, causal, on odd threads;
    # (64, 1500), 6 heads, on even ones
    t_q, t_kv, h = (100, 137, 3) if i & 1 else (64, 1500, 6)
    dm = h * 64
    c["hs"] = dict(q=W.normal((t_q, dm), 700 + 10 * i), k=W.normal((t_kv, dm), 701 + 10 * i),
                   v=W.normal((t_kv, dm), 702 + 10 * i), t_q=t_q, t_kv=t_kv, h=h, dm=dm,
                   causal=bool(i & 1))
    d = c["hs"]
    d["ref"] = _oracle_fa2(orc, d["q"], d["k"], d["v"], t_q, t_kv, h, dm, d["causal"])
    # device-resident prefill, f16: 2 windows x 4 heads x 300 frames on odd
    # threads, one whisper-base window (8 heads x 1500 frames) on even ones
    B, H, T = (2, 4, 300) if i & 1 else (1, 8, 1500)
    dmp = H * 64
    q = W.normal((B, T, dmp), 800 + 10 * i, storage="f16")
    k = W.normal((B, T, dmp), 801 + 10 * i, storage="f16")
    v = W.normal((B, T, dmp), 802 + 10 * i, storage="f16")
    ref = np.stack([_oracle_fa2(orc, q[b], k[b], v[b], T, T, H, dmp) for b in range(B)])
    c["pf"] = dict(q=q, k=k, v=v, B=B, H=H, T=T, dm=dmp, ref=ref)
    # cross decode, beam 5 over 700 f16 frames, 8 heads
    Hd, n_audio, beams = 8, 700, 5
    dmd = Hd * 64
    kc = W.normal((n_audio, dmd), 900 + 10 * i, storage="f16")
    vc = W.normal((n_audio, dmd), 901 + 10 * i, storage="f16")
    qd = W.normal((beams, dmd), 902 + 10 * i)
    refd = np.zeros((beams, dmd), np.float32)
    for b in range(beams):
        orc.single_token_mha_d64(qd[b].copy(), kc.ravel().copy(), vc.ravel().copy(), n_audio,
                                 Hd, dmd, refd[b])
    c["dec"] = dict(k=kc, v=vc, q=qd, H=Hd, n_audio=n_audio, beams=beams, dm=dmd, ref=refd)
    return c


def test_four_threads_four_contexts_at_once(wrs, orc):
    from wrs_amd import workloads as W
    note(f"{N_THREADS} host threads, one context each: host-slice, prefill and decode at once")
    cases = [_case(orc, W, i) for i in range(N_THREADS)]
    failures: list[str] = []
    stop = threading.Event()
    start = threading.Barrier(N_THREADS)

    def worker(i):
        c = cases[i]
        ctx = wrs.Context(0)  # its own stream
        try:
            hs, pf, dc = c["hs"], c["pf"], c["dec"]
            pq, pk, pv = (dev(x, torch.float16) for x in (pf["q"], pf["k"], pf["v"]))
            pout = torch.empty((pf["B"], pf["T"], pf["dm"]), device="cuda")
            lay = wrs.token_major(pf["T"], pf["dm"], 64)
            ar = wrs.KvArena(1, 1, dc["H"], 16, dc["n_audio"], ctx=ctx)
            ar.set_cross(0, dev(dc["k"]), dev(dc["v"]))
            dq = dev(dc["q"])
            dout = torch.empty((dc["beams"], dc["dm"]), device="cuda")
            ctx.synchronize()
            torch.cuda.synchronize()
            start.wait()
            for r in range(ROUNDS):
                if stop.is_set():
                    break
                pout.fill_(float("nan"))
                dout.fill_(float("nan"))
                torch.cuda.synchronize()
                # asynchronous device work first, then the synchronous host slice
                wrs.prefill(pq, pk, pv, pout, batch=pf["B"], n_heads=pf["H"], t_q=pf["T"],
                            t_kv=pf["T"], d_head=64, q_layout=lay, kv_layout=lay,
                            out_layout=lay, ctx=ctx)
                ar.decode_cross(0, dq, dout)
                out = np.full((hs["t_q"], hs["dm"]), np.nan, np.float32)
                wrs.flash_attention_2(hs["q"], hs["k"], hs["v"], hs["t_q"], hs["t_kv"], hs["h"],
                                      hs["dm"], hs["causal"], out, ctx=ctx)
                ctx.synchronize()
                e_hs = float(np.abs(out - hs["ref"]).max())
                e_pf = float(np.abs(host(pout) - pf["ref"]).max())
                e_dc = float(np.abs(host(dout) - dc["ref"]).max())
                if not (e_hs <= 1e-5 and e_pf <= 2e-3 and e_dc <= 2e-3):
                    failures.append(f"thread {i} round {r}: host-slice {e_hs:.3g}, "
                                    f"prefill {e_pf:.3g}, decode {e_dc:.3g}")
                    stop.set()
                    break
            ar.close()
        except Exception as exc:  # noqa: BLE001 -- reported below
            failures.append(f"thread {i}: {type(exc).__name__}: {exc}")
            stop.set()
        finally:
            ctx.close()

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(N_THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not failures, "; ".join(failures)
