"""ctypes binding of libwrs_attn.so (the C ABI declared in include/wrs_attn.h).

The library is the only compute path of this package: if it is missing, every
entry point raises instead of computing anything on the CPU.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
# WRS_ATTN_LIB selects another build of the library (same C ABI) for A/B
# measurements; by default the one built in the package's lib/ directory.
# Loading another build is announced on stderr.
DEFAULT_LIB_PATH = PKG_DIR / "lib" / "libwrs_attn.so"
LIB_PATH = Path(os.environ.get("WRS_ATTN_LIB") or DEFAULT_LIB_PATH)
HEADER_PATH = PKG_DIR.parent / "include" / "wrs_attn.h"

WRS_OK = 0
WRS_EINVAL = -1
WRS_ENOMEM = -2
WRS_EHIP = -3
WRS_EUNSUPPORTED = -4
WRS_ERANGE = -5
WRS_ECAPTURE = -6
WRS_EBUSY = -7

WRS_F32 = 0
WRS_F16 = 1
WRS_BF16 = 2


class Reserve(ctypes.Structure):
    """wrs_reserve: the largest calls a context serves (scratch sized up front)."""

    _fields_ = [(n, ctypes.c_size_t) for n in (
        "n_heads", "decode_rows", "decode_keys", "capture_tokens", "capture_keys",
        "linear_tokens", "linear_n_in")]


class Layout(ctypes.Structure):
    """wrs_layout: strides (elements) of a [batch][head][token][d] view."""

    _fields_ = [("batch_stride", ctypes.c_int64), ("head_stride", ctypes.c_int64),
                ("row_stride", ctypes.c_int64)]


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int
_szp = ctypes.POINTER(ctypes.c_size_t)
_LP = ctypes.POINTER(Layout)

_SIGNATURES = {
    "wrs_attn_create": (_int, [_int, ctypes.POINTER(_vp)]),
    "wrs_attn_destroy": (None, [_vp]),
    "wrs_attn_set_stream": (_int, [_vp, _vp]),
    "wrs_attn_get_stream": (_vp, [_vp]),
    "wrs_attn_set_schedule": (_int, [_vp, _int, _int]),
    "wrs_attn_synchronize": (_int, [_vp]),
    "wrs_attn_last_error": (ctypes.c_char_p, [_vp]),
    "wrs_attn_status_string": (ctypes.c_char_p, [_int]),
    "wrs_attn_reserve": (_int, [_vp, ctypes.POINTER(Reserve)]),
    "wrs_stream_read": (_int, [_vp, _vp, _sz, _vp, _sz]),
    "wrs_stream_read_shape": (_int, [_vp, _vp, _sz, _int, _int, _vp, _sz]),
    "wrs_flash_attention_2": (_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz, _int,
                                     _vp, _sz]),
    "wrs_multi_head_attention": (_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz,
                                        _int, _vp, _sz]),
    "wrs_single_token_mha_d64": (_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _vp,
                                        _sz]),
    "wrs_mha_with_cache": (_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp,
                                  _sz]),
    "wrs_attn_prefill": (_int, [_vp, _int, _vp, _LP, _int, _vp, _LP, _vp, _LP, _vp, _LP, _sz, _sz,
                                _sz, _sz, _sz, _int, _sz]),
    "wrs_kv_create": (_int, [_vp, _sz, _sz, _sz, _sz, _sz, ctypes.POINTER(_vp)]),
    "wrs_kv_create_dtype": (_int, [_vp, _sz, _sz, _sz, _sz, _sz, _int, ctypes.POINTER(_vp)]),
    "wrs_kv_dtype": (_int, [_vp, ctypes.POINTER(_int)]),
    "wrs_kv_destroy": (None, [_vp]),
    "wrs_kv_clear": (_int, [_vp]),
    "wrs_kv_clear_slot": (_int, [_vp, _sz]),
    "wrs_kv_invalidate_cross": (_int, [_vp]),
    "wrs_kv_ensure_slots": (_int, [_vp, _sz]),
    "wrs_kv_copy_slot": (_int, [_vp, _sz, _sz]),
    "wrs_kv_slot_len": (_int, [_vp, _sz, _szp]),
    "wrs_kv_set_len": (_int, [_vp, _sz, _sz]),
    "wrs_kv_slide_to_fit": (_int, [_vp, _sz, _sz, _sz, _szp]),
    "wrs_kv_append": (_int, [_vp, _sz, _sz, _vp, _vp, _sz, _int]),
    "wrs_kv_advance": (_int, [_vp, _sz, _sz]),
    "wrs_kv_set_cross": (_int, [_vp, _sz, _vp, _vp, _sz, _int]),
    "wrs_kv_cross_len": (_int, [_vp, _sz, _szp]),
    "wrs_kv_self_planes": (_int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _szp]),
    "wrs_kv_cross_planes": (_int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "wrs_attn_decode_self": (_int, [_vp, _vp, _sz, _szp, _sz, _vp, _vp]),
    "wrs_attn_decode_cross": (_int, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "wrs_attn_decode_cross_noalloc": (_int, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "wrs_attn_prefill_self": (_int, [_vp, _vp, _sz, _sz, _vp, _sz, _vp]),
    "wrs_attn_prefill_cross": (_int, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "wrs_attn_prefill_cross_lse": (_int, [_vp, _vp, _sz, _vp, _sz, _vp, _vp]),
    "wrs_linear": (_int, [_vp, _int, _vp, _sz, ctypes.c_int64, _vp, _vp, _sz, _sz, _sz, _int,
                          _vp, _sz, ctypes.c_int64, ctypes.c_int64]),
    "wrs_linear_group": (_int, [_vp, _int, _vp, _sz, ctypes.c_int64, _sz, ctypes.POINTER(_vp),
                                ctypes.POINTER(_vp), _sz, _sz, _sz, _int, ctypes.POINTER(_vp),
                                _szp, ctypes.c_int64, ctypes.c_int64]),
    "wrs_linear_fused": (_int, [_vp, _vp, _sz, ctypes.c_int64, _vp, _vp, ctypes.c_float, _sz,
                                ctypes.POINTER(_vp), ctypes.POINTER(_vp), _sz, _sz, _sz, _int, _int,
                                ctypes.POINTER(_vp), _szp, ctypes.c_int64, ctypes.c_int64]),
    "wrs_layer_norm": (_int, [_vp, _vp, _sz, _vp, _vp, ctypes.c_float, _sz, _sz, _int, _vp, _sz]),
    "wrs_gelu_inplace": (_int, [_vp, _vp, _sz]),
    "wrs_kv_set_cross_proj": (_int, [_vp, _int, _vp, _sz, ctypes.c_int64, _sz,
                                     ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                     ctypes.POINTER(_vp)]),
    "wrs_attn_capture_cross_heads": (_int, [_vp, _vp, _sz, _vp, _sz, _szp, _szp, _sz, _sz, _sz,
                                            _vp, _sz]),
    "wrs_attn_capture_cross_heads_lse": (_int, [_vp, _vp, _sz, _vp, _sz, _szp, _szp, _sz, _sz, _sz,
                                            _vp, _sz, _vp]),
}

_lib = None


class ExtensionMissing(RuntimeError):
    pass


def header_symbols() -> list[str]:
    """Function names declared in include/wrs_attn.h."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wrs_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ExtensionMissing(
                f"HIP extension not built: {LIB_PATH} is missing (run __graft_entry__.build())")
        if LIB_PATH.resolve() != DEFAULT_LIB_PATH.resolve():
            import sys
            print(f"[wrs_amd] WRS_ATTN_LIB: loading {LIB_PATH}, not {DEFAULT_LIB_PATH}",
                  file=sys.stderr, flush=True)
        L = ctypes.CDLL(str(LIB_PATH))
        other = LIB_PATH.resolve() != DEFAULT_LIB_PATH.resolve()
        for name, (res, args) in _SIGNATURES.items():
            if other and not hasattr(L, name):
                # another build for an A/B measurement may predate an entry point
                import sys
                print(f"[wrs_amd] {LIB_PATH} lacks {name}", file=sys.stderr, flush=True)
                continue
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def status_string(code: int) -> str:
    return lib().wrs_attn_status_string(code).decode()
