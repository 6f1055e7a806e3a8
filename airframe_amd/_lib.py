"""ctypes binding of libturboshimmy.so (declared in include/turboshimmy.h).

Loading never falls back to anything: if the built library is missing, ``load()`` raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libturboshimmy.so")

TS_OK = 0
TS_ERR_INVALID = -1
TS_ERR_OVERFLOW = -2
TS_ERR_UNSUPPORTED = -3
TS_ERR_HIP = -4
TS_ERR_NOMEM = -5
TS_ERR_WORKSPACE = -6

# Every symbol the header declares, with (restype, argtypes).
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f = ctypes.c_float


class KvDesc(ctypes.Structure):
    _fields_ = [("n_layers", _i32), ("n_seq", _i32), ("n_head_kv", _i32), ("head_dim", _i32),
                ("max_seq", _i32)]


SIGNATURES = {
    "ts_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "ts_rope_table_host": (ctypes.c_int, [_vp, _i32, _i32, _f, _f]),
    "ts_rope_create": (ctypes.c_int, [_i32, _i32, _f, _f, ctypes.POINTER(_vp)]),
    "ts_weights_src_bytes": (ctypes.c_int, [_i32, ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint64)]),
    "ts_weights_to_f16": (ctypes.c_int, [_i32, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp]),
    "ts_rope_table_host_yarn": (ctypes.c_int, [_vp, _i32, _i32, _f, _f, _f, _f]),
    "ts_rope_create_yarn": (ctypes.c_int, [_i32, _i32, _f, _f, _f, _f, ctypes.POINTER(_vp)]),
    "ts_rope_destroy": (ctypes.c_int, [_vp]),
    "ts_rope_info": (ctypes.c_int, [_vp, ctypes.POINTER(_vp), _i32p, _i32p]),
    "ts_kv_bytes": (ctypes.c_int, [ctypes.POINTER(KvDesc), _u64p]),
    "ts_kv_create": (ctypes.c_int, [ctypes.POINTER(KvDesc), ctypes.POINTER(_vp)]),
    "ts_kv_destroy": (ctypes.c_int, [_vp]),
    "ts_kv_desc_get": (ctypes.c_int, [_vp, ctypes.POINTER(KvDesc)]),
    "ts_kv_seq_len": (ctypes.c_int, [_vp, _i32, _i32p]),
    "ts_kv_max_len": (ctypes.c_int, [_vp, _i32p]),
    "ts_kv_increment": (ctypes.c_int, [_vp, _i32, _vp]),
    "ts_kv_set_seq_len": (ctypes.c_int, [_vp, _i32, _i32, _vp]),
    "ts_kv_reset": (ctypes.c_int, [_vp, _vp]),
    "ts_kv_reset_seq": (ctypes.c_int, [_vp, _i32, _vp]),
    "ts_kv_export": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "ts_kv_set_qk_norm": (ctypes.c_int, [_vp, _i32, _vp, _vp, _f]),
    "ts_kv_window_base": (ctypes.c_int, [_vp, _i32, _i32p]),
    "ts_kv_advance_window_base": (ctypes.c_int, [_vp, _i32, _i32, _vp]),
    "ts_kv_shift_workspace": (ctypes.c_int, [_vp, _u64p]),
    "ts_kv_shift": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, ctypes.c_uint64, _vp]),
    "ts_append_quant": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i32, _vp, _vp]),
    "ts_requant_all": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i32, _i32, _vp, _vp]),
    "ts_attn_decode_workspace": (ctypes.c_int, [_vp, _i32, _u64p]),
    "ts_attn_decode": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _f, _vp, _vp, ctypes.c_uint64, _vp]),
    "ts_attn_decode_append": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _i32, _vp, _f, _vp, _vp,
                                             ctypes.c_uint64, _vp]),
    "ts_attn_decode_append_advance": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _i32, _vp, _f, _vp, _vp,
                                             ctypes.c_uint64, _vp]),
    "ts_attn_decode_append_noalloc": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _i32, _vp, _f, _vp, _vp]),
    "ts_attn_prefill": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i32, _vp, _f, _vp, _vp]),
    "ts_qkv_workspace": (ctypes.c_int, [_vp, _i32, _i32, _i32, _u64p]),
    "ts_qkv_gguf_workspace": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _u64p]),
    "ts_qkv_append_gguf": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp,
                                          _vp, _vp, _vp, ctypes.c_uint64, _vp]),
    "ts_attn_out_proj_gguf_workspace": (ctypes.c_int, [_i32, _i32, _i32, _i32, _u64p]),
    "ts_attn_out_proj_gguf": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp, ctypes.c_uint64,
                                             _vp]),
    "ts_qkv_append": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp,
                                     _vp, _vp, _vp, ctypes.c_uint64, _vp]),
    "ts_attn_out_proj_workspace": (ctypes.c_int, [_i32, _i32, _i32, _u64p]),
    "ts_attn_out_proj": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, ctypes.c_uint64,
                                        _vp]),
    "ts_qkv_append_x2": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp,
                                        _vp, _vp, _vp, ctypes.c_uint64, _vp]),
    "ts_attn_out_proj_x2": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, ctypes.c_uint64,
                                           _vp]),
    "ts_weights_to_f16x2": (ctypes.c_int, [_i32, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp]),
}

_lib = None


class TsError(RuntimeError):
    def __init__(self, fn: str, code: int):
        self.code = code
        msg = load().ts_status_string(code).decode() if _lib is not None else str(code)
        super().__init__(f"{fn} failed: {msg} ({code})")


def load():
    """Load the built library (build it first with ``python -m airframe_amd.build``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: the HIP extension has not been built "
                "(python -m airframe_amd.build); there is no fallback path")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, code: int) -> None:
    if code != TS_OK:
        raise TsError(fn, code)
