"""GPU parity of the row and element kernels around the projections:
layer_norm (crates/tensor/src/ops/norm.rs:116-143) and gelu_inplace
(crates/tensor/src/ops/gelu.rs:11-23), through the C ABI against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import dev, host, note

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx(wrs):
    c = wrs.Context(0)
    c.use_torch_stream()
    return c


@pytest.mark.parametrize("n_tokens,d", [(1, 384), (5, 1280), (1500, 1280), (7, 5120), (3, 260)])
def test_layer_norm_matches_oracle(wrs, orc, ctx, n_tokens, d):
    note(f"layer_norm T={n_tokens} d={d}")
    rng = np.random.default_rng(d + n_tokens)
    x = (2.0 * rng.standard_normal((n_tokens, d)) + 0.7).astype(np.float32)
    g = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    out = torch.full((n_tokens, d), float("nan"), device="cuda")
    wrs.layer_norm(dev(x), dev(g), dev(b), 1e-5, out, ctx=ctx)
    ref = np.zeros(n_tokens * d, np.float32)
    orc.layer_norm(x.ravel(), g, b, 1e-5, n_tokens, d, ref)
    ref = ref.reshape(n_tokens, d)
    # f32 sums in another order: a few ulp of the normalized value, times gamma
    tol = 4e-6 * (np.abs(g) * 6.0 + 1.0)
    assert (np.abs(host(out) - ref) <= tol).all()


@pytest.mark.parametrize("out_dt", [torch.float16, torch.bfloat16])
def test_layer_norm_rounded_output(wrs, orc, ctx, out_dt):
    note(f"layer_norm out {out_dt}")
    n_tokens, d = 64, 1280
    rng = np.random.default_rng(5)
    x = rng.standard_normal((n_tokens, d)).astype(np.float32)
    g = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    out = torch.zeros((n_tokens, d), dtype=out_dt, device="cuda")
    wrs.layer_norm(dev(x), dev(g), dev(b), 1e-5, out, ctx=ctx)
    ref = np.zeros(n_tokens * d, np.float32)
    orc.layer_norm(x.ravel(), g, b, 1e-5, n_tokens, d, ref)
    rt = torch.from_numpy(ref.reshape(n_tokens, d)).to(out_dt).float().numpy()
    got = out.float().cpu().numpy()
    rel = 2.0 ** -10 if out_dt == torch.float16 else 2.0 ** -7
    assert (np.abs(got - rt) <= np.abs(rt) * rel + 1e-4).all()
    assert np.mean(got == rt) > 0.99


def test_layer_norm_constant_row_is_beta(wrs, ctx):
    note("layer_norm constant row")
    d = 512
    b = np.random.default_rng(9).standard_normal(d).astype(np.float32)
    out = torch.zeros((2, d), device="cuda")
    wrs.layer_norm(torch.full((2, d), -4.5, device="cuda"), dev(np.ones(d, np.float32)), dev(b),
                   1e-5, out, ctx=ctx)
    assert np.array_equal(host(out), np.stack([b, b]))


@pytest.mark.parametrize("n", [1, 7, 4096, 5 * 5120, 1500 * 5120 + 3])
def test_gelu_matches_oracle(wrs, orc, ctx, n):
    note(f"gelu n={n}")
    x = (4.0 * np.random.default_rng(n).standard_normal(n)).astype(np.float32)
    t = dev(x)
    wrs.gelu_inplace(t, ctx=ctx)
    ref = x.copy()
    orc.gelu_inplace(ref)
    got = host(t)
    # tanhf on either side within a few ulp
    assert (np.abs(got - ref) <= 4e-7 * np.maximum(np.abs(ref), 1.0)).all()
