"""ctypes binding of ``libbitgpu_attn.so`` (the C ABI declared in include/bitgpu_attn.h).

The library is built in-tree by ``python -m bitgpu_amd.build``. Loading fails loudly when it is
missing: there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libbitgpu_attn.so")

BG_OK = 0
BG_E_INVALID = -1
BG_E_OOM = -2
BG_E_DEVICE = -3
BG_E_UNSUPPORTED = -4
BG_E_STATE = -5

BG_KV_F32, BG_KV_F16, BG_KV_Q8 = 0, 1, 2
BG_K, BG_V, BG_KSCALE, BG_VSCALE = 0, 1, 2, 3
BG_ROPE_SLOT, BG_ROPE_ABSOLUTE = 0, 1

KV_DTYPES = {"f32": BG_KV_F32, "f16": BG_KV_F16, "q8": BG_KV_Q8}

# (name, restype, argtypes) for every exported symbol of include/bitgpu_attn.h
_i32, _f32, _f64, _vp = C.c_int32, C.c_float, C.c_double, C.c_void_p
_pi32 = C.POINTER(C.c_int32)
SIGNATURES = [
    ("bg_last_error_message", C.c_char_p, []),
    ("bg_version", C.c_char_p, []),
    ("bg_rope_tables", _i32, [_f64, _i32, _i32, _f64, _i32, _vp, _vp]),
    ("bg_evict_plan", _i32, [_i32, _i32, _i32, _i32, _pi32, _pi32, _pi32]),
    ("bg_ring_map", _i32, [_i32, _i32, _i32, _i32, _pi32]),
    ("bg_stream_sync", _i32, [_vp]),
    ("bg_decode_plan", _i32, [_i32] * 8 + [_pi32]),
    ("bg_diag_stream_read", _i32, [_vp, C.c_size_t, _i32, _i32, _vp, _vp]),
    ("bg_debug_merge_hooks", _i32, [_i32, _i32]),
    ("bg_stream_create", _i32, [C.POINTER(_vp)]),
    ("bg_stream_destroy", _i32, [_vp]),
    ("bg_event_create", _i32, [C.POINTER(_vp)]),
    ("bg_event_record", _i32, [_vp, _vp]),
    ("bg_event_elapsed_us", _i32, [_vp, _vp, C.POINTER(_f32)]),
    ("bg_event_destroy", _i32, [_vp]),
    ("bg_kv_create", _i32, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, C.POINTER(_vp)]),
    ("bg_kv_destroy", _i32, [_vp]),
    ("bg_kv_capacity", _i32, [_vp, _pi32]),
    ("bg_kv_grow", _i32, [_vp, _i32, _vp]),
    ("bg_kv_set_q8_block", _i32, [_vp, _i32]),
    ("bg_kv_set_rope", _i32, [_vp, _vp, _vp, _i32, _i32]),
    ("bg_kv_write", _i32, [_vp, _i32, _i32, _vp, _i32, _i32, _vp]),
    ("bg_qkv_prologue", _i32, [_vp, _i32, _vp, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _f32,
                               _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    ("bg_gemv_split", _i32, [_vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    ("bg_gemv_resid", _i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp]),
    ("bg_qkv_proj_prologue", _i32, [_vp, _i32, _vp, _i32, _vp, _vp, _i32, _vp, _vp, _f32, _vp, _vp, _i32, _i32,
                                     _i32, _i32, _vp, _vp]),
    ("bg_attention", _i32, [_vp, _i32, _vp, _i32, _i32, _i32, _f32, _vp, _i32, _vp, _vp]),
    ("bg_attention_noalloc", _i32, [_vp, _i32, _vp, _i32, _i32, _i32, _f32, _vp, _i32, _vp, _vp]),
    ("bg_attention_reserve", _i32, [_vp, _i32, _i32]),
    ("bg_kv_evict", _i32, [_vp, _i32, _i32, _pi32]),
    ("bg_kv_evict_for", _i32, [_vp, _i32, _i32, _pi32]),
    ("bg_kv_ring_state", _i32, [_vp, _pi32, C.POINTER(C.c_int64)]),
    ("bg_kv_ring_reset", _i32, [_vp, C.c_int64]),
    ("bg_kv_region_bytes", _i32, [_vp, _i32, _i32, C.POINTER(C.c_size_t)]),
    ("bg_kv_export_rows", _i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    ("bg_kv_import_rows", _i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
]


class BitgpuError(RuntimeError):
    """A failed C-ABI call; the message is the library's (``bitgpu: ...``, src/errors.ts style)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class GpuOutOfMemoryError(BitgpuError):
    """Device allocation failed (the reference's GpuOutOfMemoryError, src/errors.ts:14-19)."""


_lib = None


def lib():
    """Load (once) and return the library; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"bitgpu_amd: HIP library not found at {LIB_PATH}; build it with `python -m bitgpu_amd.build`")
        h = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(rc: int) -> None:
    if rc == BG_OK:
        return
    msg = lib().bg_last_error_message().decode("utf-8", "replace")
    if rc == BG_E_OOM:
        raise GpuOutOfMemoryError(rc, msg)
    raise BitgpuError(rc, msg)
