"""Number-format facts the 16-bit prefill kernel relies on, checked over every
bf16 bit pattern, and the kernel-name patterns the bench's traffic pass uses.

* bf16 -> f16 (widen to f32, round to nearest even) is exact for every bf16
  value of magnitude in [2^-14, 65536), and inf for every finite one at or
  above 65536: the kernel's in-LDS V conversion, and the range its non-finite
  output check hands to the f32 recompute.
* The check's predicate ((bits & 0x7f800000) == 0x7f800000 on the lane's sum
  of outputs) holds exactly for inf and NaN.
"""
from __future__ import annotations

import importlib.util
import re
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def _all_bf16() -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    return bits.view(np.float32)


def test_bf16_to_f16_is_exact_inside_the_normal_range():
    x = _all_bf16()
    finite = np.isfinite(x)
    mag = np.abs(x)
    normal = finite & (mag >= 2.0 ** -14) & (mag < 65536.0)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(h[normal], x[normal])
    # the largest bf16 below 65536 is 65280, which f16 holds
    assert h[np.argmax(np.where(normal, mag, 0))] == 65280.0


def test_bf16_to_f16_overflows_exactly_from_65536():
    x = _all_bf16()
    finite = np.isfinite(x)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16).astype(np.float32)
    big = finite & (np.abs(x) >= 65536.0)
    assert np.isinf(h[big]).all() and (np.sign(h[big]) == np.sign(x[big])).all()
    assert np.isfinite(h[finite & ~big]).all()


def test_bf16_subnormal_range_error_is_below_f16_spacing():
    # below 2^-14 the f16 result is a subnormal: absolute error <= 2^-25
    x = _all_bf16()
    small = np.isfinite(x) & (np.abs(x) < 2.0 ** -14)
    h = x[small].astype(np.float16).astype(np.float64)
    assert np.abs(h - x[small].astype(np.float64)).max() <= 2.0 ** -25


def test_nonfinite_predicate_is_exactly_inf_or_nan():
    x = _all_bf16()  # covers every exponent, both signs, inf and NaN patterns
    bits = x.view(np.uint32)
    pred = (bits & np.uint32(0x7F800000)) == np.uint32(0x7F800000)
    assert np.array_equal(pred, ~np.isfinite(x))


def test_inf_minus_inf_sum_is_flagged():
    with np.errstate(invalid="ignore"):
        s = np.float32(np.inf) + np.float32(-np.inf) + np.float32(1.0)
    assert (np.float32(s).view(np.uint32) & 0x7F800000) == 0x7F800000


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_traffic_patterns_match_mangled_and_demangled_names():
    legs = _bench().TRAFFIC_LEGS
    names = {
        "encoder": ["_ZN3wrs12_GLOBAL__N_115fa2_prefill_d64IDF16bEEvNS_11PrefillArgsEi",
                    "void wrs::(anonymous namespace)::fa2_prefill_d64<__bf16>(wrs::PrefillArgs, int)"],
        "encoder_base": ["_ZN3wrs12_GLOBAL__N_115fa2_prefill_d64IDF16_EEvNS_11PrefillArgsEi",
                         "void wrs::(anonymous namespace)::fa2_prefill_d64<_Float16>(wrs::PrefillArgs, int)"],
        "decode": ["void wrs::(anonymous namespace)::decode_f16<5, 8>(wrs::DecodeArgs)"],
        "decode_self": ["void wrs::(anonymous namespace)::decode_f16<1, 16>(wrs::DecodeArgs)"],
        "capture": ["void wrs::(anonymous namespace)::capture_cross_f16<2>(wrs::CaptureArgs, int, int)"],
        "capture_two_pass": ["void wrs::(anonymous namespace)::capture_cross_f16<0>(wrs::CaptureArgs, int, int)",
                             "_ZN3wrs12_GLOBAL__N_117capture_cross_f16ILi1EEEvNS_11CaptureArgsEii"],
    }
    for leg, ns in names.items():
        for n in ns:
            hits = [k for k, (pat, _) in legs.items() if re.search(pat, n)]
            assert hits == [leg], (n, hits)
