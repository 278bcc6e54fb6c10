"""Synthetic Whisper-shaped attention workloads (seeded, no model weights).

Shapes come from the reference's model hyper-parameters (n_audio_ctx 1500,
n_text_ctx 448, d_head 64; crates/model/src/header.rs:36-50). Values are
N(0, sigma^2) from numpy's PCG64 seeded per tensor, rounded to the storage
type with round-to-nearest-even. Every generator returns float32 arrays whose
values are exactly representable in that storage type, so the same numbers
feed the GPU (as f16/bf16) and the CPU reference (widened exactly to f32).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SEED = 0x5EED_1234


def _round(x: np.ndarray, storage: str) -> np.ndarray:
    if storage == "f32":
        return x.astype(np.float32)
    if storage == "f16":
        return x.astype(np.float16).astype(np.float32)
    if storage == "bf16":
        # round-to-nearest-even to the top 16 bits of the f32 pattern
        b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
        r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        return r.view(np.float32)
    raise ValueError(storage)


def normal(shape, stream: int, sigma: float = 1.0, storage: str = "f32",
           seed: int = SEED) -> np.ndarray:
    rng = np.random.default_rng(seed + stream)
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if sigma != 1.0:
        x *= np.float32(sigma)
    return _round(x, storage)


def outlier_channels(d_model: int, n: int, seed: int = SEED) -> np.ndarray:
    return np.random.default_rng(seed ^ 0x0171).permutation(d_model)[:n]


@dataclass(frozen=True)
class Encoder:
    """Encoder self-attention: `batch` independent windows of [T][H*64] rows."""

    name: str
    batch: int
    n_heads: int
    t: int
    storage: str  # f32 | f16 | bf16
    sigma: float = 1.0
    outliers: int = 0  # channels scaled x8 before rounding (same set for Q, K, V)
    qk_prescale: float = 1.0  # Q and K multiplied by this after sampling

    @property
    def d_model(self) -> int:
        return self.n_heads * 64

    def flops(self) -> float:
        # 4*B*H*T^2*d, crates/tensor/tests/bench_flash_attention_tiled.rs:214
        return 4.0 * self.batch * self.n_heads * self.t * self.t * 64

    def inputs(self, batch: int | None = None):
        b = self.batch if batch is None else batch
        shape = (b, self.t, self.d_model)
        ch = outlier_channels(self.d_model, self.outliers) if self.outliers else None
        out = []
        for stream in (1, 2, 3):
            rng = np.random.default_rng(SEED + stream)
            x = rng.standard_normal(size=(self.batch, self.t, self.d_model), dtype=np.float32)[:b]
            if self.sigma != 1.0:
                x *= np.float32(self.sigma)
            if ch is not None:
                x[:, :, ch] *= np.float32(8.0)
            if stream in (1, 2) and self.qk_prescale != 1.0:
                x *= np.float32(self.qk_prescale)
            out.append(_round(x, self.storage).reshape(shape))
        return tuple(out)


@dataclass(frozen=True)
class CrossDecode:
    """Beam decode against the shared encoder K/V of `n_layers` layers."""

    name: str
    beams: int
    n_heads: int
    n_audio: int
    n_layers: int

    @property
    def d_model(self) -> int:
        return self.n_heads * 64

    def bytes_per_layer(self) -> int:
        # unique K+V f16 read once for all beams, plus f32 Q in and O out
        return 2 * self.n_heads * self.n_audio * 64 * 2 + 2 * self.beams * self.d_model * 4

    def q(self, layer: int) -> np.ndarray:
        return normal((self.beams, self.d_model), 100 + layer)

    def kv(self, layer: int):
        k = normal((self.n_audio, self.d_model), 1000 + 2 * layer, storage="f16")
        v = normal((self.n_audio, self.d_model), 1001 + 2 * layer, storage="f16")
        return k, v


@dataclass(frozen=True)
class SelfDecode:
    """One decode step of causal self-attention, one slot per beam."""

    name: str
    beams: int
    n_heads: int
    ctx: int  # valid cache length including the step's own row
    max_ctx: int = 448

    @property
    def d_model(self) -> int:
        return self.n_heads * 64

    def bytes(self) -> int:
        return self.beams * 2 * self.ctx * self.n_heads * 64 * 2 + 2 * self.beams * self.d_model * 4

    def q(self) -> np.ndarray:
        return normal((self.beams, self.d_model), 200)

    def kv(self, slot: int):
        k = normal((self.ctx, self.d_model), 2000 + 2 * slot, storage="f16")
        v = normal((self.ctx, self.d_model), 2001 + 2 * slot, storage="f16")
        return k, v


@dataclass(frozen=True)
class AlignmentCapture:
    """DTW alignment pass of one segment: the cross-attention weights of the
    preset's (text layer, head) pairs for every token of the segment."""

    name: str
    n_tokens: int
    n_heads: int
    n_audio: int
    n_layers: int
    heads: tuple  # ((layer, head), ...)

    @property
    def d_model(self) -> int:
        return self.n_heads * 64

    def layers(self) -> list[int]:
        return sorted({l for l, _ in self.heads})

    def pairs(self, layer: int) -> list[tuple[int, int]]:
        return [(slot, h) for slot, (l, h) in enumerate(self.heads) if l == layer]

    def bytes_per_pair(self) -> int:
        # the head's f16 K plane, its f32 query slices, the f32 weights written
        return (self.n_audio * 64 * 2 + self.n_tokens * 64 * 4
                + self.n_tokens * self.n_audio * 4)

    def q(self, layer: int) -> np.ndarray:
        return normal((self.n_tokens, self.d_model), 500 + layer)

    def k(self, layer: int) -> np.ndarray:
        return normal((self.n_audio, self.d_model), 3000 + layer, storage="f16")


@dataclass(frozen=True)
class Projection:
    """LinearWeight::linear with f16 weights over a batch of token rows."""

    name: str
    n_tokens: int
    n_in: int
    n_out: int
    x_storage: str  # f32 | f16

    def flops(self) -> float:
        return 2.0 * self.n_tokens * self.n_in * self.n_out

    def x(self) -> np.ndarray:
        return normal((self.n_tokens, self.n_in), 600, storage=self.x_storage)

    def w(self) -> np.ndarray:
        return normal((self.n_out, self.n_in), 601, sigma=self.n_in ** -0.5,
                      storage="f16").astype(np.float16)

    def bias(self) -> np.ndarray:
        return normal((self.n_out,), 602, sigma=0.1)


# crates/whisper/src/dtw.rs AlignmentHeadsPreset::LargeV3
LARGE_V3_ALIGNMENT_HEADS = ((7, 0), (10, 17), (12, 18), (13, 12), (16, 1), (17, 14), (19, 11),
                            (21, 4), (24, 1), (25, 6))

TINY_ENCODER = Encoder("whisper-tiny encoder self-attention, f32", 1, 6, 1500, "f32",
                       qk_prescale=64.0 ** -0.25)
BASE_ENCODER = Encoder("whisper-base encoder self-attention x4 windows, f16", 4, 8, 1500, "f16")
# one 30 s window per call, as the reference's encoder runs it
BASE_ENCODER_1 = Encoder("whisper-base encoder self-attention, one window, f16", 1, 8, 1500,
                         "f16")
LARGE_ENCODER_1 = Encoder("whisper-large-v3 encoder self-attention, one window, bf16 outliers",
                          1, 20, 1500, "bf16", sigma=0.5, outliers=13)
SMALL_SELF_DECODE = SelfDecode("whisper-small self-attention decode, beam 5", 5, 12, 224)
LARGE_CROSS_DECODE = CrossDecode("whisper-large-v3 cross-attention decode, beam 5", 5, 20, 1500,
                                 32)
LARGE_ENCODER = Encoder("whisper-large-v3 encoder self-attention x16 windows, bf16 outliers", 16,
                        20, 1500, "bf16", sigma=0.5, outliers=13)
SELF_DECODE_SWEEP = (32, 64, 128, 224, 256, 384, 448)
# 124 text tokens + SOT, language, NOT and EOT (transcribe.rs:1403-1411)
LARGE_DTW_CAPTURE = AlignmentCapture("whisper-large-v3 DTW alignment-head capture, 128 tokens",
                                     128, 20, 1500, 32, LARGE_V3_ALIGNMENT_HEADS)
# encoder.rs:275-277 for 16 windows of 1500 frames (one layer), bf16 Q/K/V out
LARGE_QKV_F16 = Projection("whisper-large-v3 encoder fused QKV projection x16 windows, f16 x",
                           16 * 1500, 1280, 3840, "f16")
LARGE_QKV_F32 = Projection("whisper-large-v3 encoder fused QKV projection x16 windows, f32 x",
                           16 * 1500, 1280, 3840, "f32")


@dataclass(frozen=True)
class DecoderWeightStream:
    """The projections of one decoder step for `beams` rows: per layer
    q, k, v, out, cross q, cross out (d x d), mlp0 (4d x d) and mlp2 (d x 4d)
    (decoder.rs:596-760), then the vocabulary projection (decoder.rs:781-783)."""

    name: str
    beams: int
    d_model: int
    n_layers: int
    n_vocab: int

    def matrices(self) -> list[tuple[int, int]]:
        d = self.d_model
        per_layer = [(d, d)] * 6 + [(4 * d, d), (d, 4 * d)]
        return per_layer * self.n_layers + [(self.n_vocab, d)]

    def weight_bytes(self) -> int:
        return sum(r * c * 2 for r, c in self.matrices())

    def launches(self) -> int:
        """q, k and v share one grouped launch per layer; every other projection
        is a launch of its own."""
        return (len(self.matrices()) - 1) - 2 * self.n_layers + 1


LARGE_DECODE_WEIGHTS = DecoderWeightStream(
    "whisper-large-v3 decoder step projections, beam 5 (32 layers + vocabulary)", 5, 1280, 32,
    51866)
