"""ctypes front end of the C oracle (ts_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the checker and
by bench.py's cpu_baseline leg.  The product library (airframe_amd) never imports it.

Array layouts are the reference's (src/backend/bindless/kv_cache.rs:26-37):
packed K/V ``[n_seq][max_seq][n_kv][hd/8]`` uint32, scales ``[n_seq][max_seq][n_kv]`` float32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libts_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no FMA contraction)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_rope_table.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        L.or_rope_table.restype = ctypes.c_int
        L.or_rope_table_yarn.argtypes = [_f32p, ctypes.c_int, ctypes.c_int] + [ctypes.c_float] * 4
        L.or_rope_table_yarn.restype = ctypes.c_int
        L.or_dequant.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_long, _f32p]
        L.or_dequant.restype = ctypes.c_int
        L.or_project_f32.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int, _f32p]
        L.or_project_f32.restype = None
        L.or_rope_rotate.argtypes = [_f32p, ctypes.c_int, _f32p]
        L.or_rope_rotate.restype = None
        L.or_quantize_row.argtypes = [_f32p, ctypes.c_int, ctypes.POINTER(ctypes.c_float), _u32p]
        L.or_quantize_row.restype = None
        L.or_dequantize_row.argtypes = [_u32p, ctypes.c_int, ctypes.c_float, _f32p]
        L.or_dequantize_row.restype = None
        L.or_append_batch.argtypes = [_u32p, _u32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                      _f32p, _i32p, ctypes.c_int, _i32p, _i32p, ctypes.c_void_p,
                                      ctypes.c_float]
        L.or_append_batch.restype = None
        L.or_attend_batch.argtypes = [_u32p, _u32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      _f32p, _f32p, _i32p, ctypes.c_int, ctypes.c_float, _f32p,
                                      ctypes.c_int, _i32p, ctypes.c_void_p, ctypes.c_float]
        L.or_attend_batch.restype = None
        L.or_attend_one.argtypes = [_u32p, _u32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_float, _f32p, ctypes.c_int, ctypes.c_void_p, ctypes.c_float]
        L.or_attend_one.restype = None
        L.or_qk_norm_row.argtypes = [_f32p, ctypes.c_int, _f32p, ctypes.c_float]
        L.or_qk_norm_row.restype = None
        L.or_shift_seq.argtypes = [_u32p, _u32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int]
        L.or_shift_seq.restype = None
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_project.argtypes = [_f32p, ctypes.c_int, ctypes.c_int,
                                 np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS"),
                                 ctypes.c_int, _f32p]
        L.or_project.restype = None
        L.or_attn_proj.argtypes = [_f32p, ctypes.c_int, ctypes.c_int,
                                   np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS"),
                                   ctypes.c_int, _f32p, ctypes.c_void_p]
        L.or_attn_proj.restype = None
        _lib = L
    return _lib


def f16_to_f32(bits: int) -> float:
    return float(lib().or_f16_to_f32(int(bits)))


def project(x: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """main_qkv's f32 dot for every (row of x, row of w): x [n, dim] f32, w [n_out, dim] f16
    bits (uint16) -> [n, n_out] f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    n, dim = x.shape
    n_out = w_bits.shape[0]
    assert w_bits.shape[1] == dim
    out = np.zeros((n, n_out), dtype=np.float32)
    lib().or_project(x, n, dim, w_bits, n_out, out)
    return out


def dequant(ggml_type: int, blob: np.ndarray, n: int) -> np.ndarray:
    """The reference's CPU dequantizers (src/core/dequant/): n f32 element values of a GGUF
    weight blob of that GGML type (n a whole number of blocks)."""
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    out = np.zeros(n, np.float32)
    if lib().or_dequant(ggml_type, blob.ctypes.data, n, out) != 0:
        raise ValueError("unsupported type or partial block")
    return out


def project_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """main_qkv's dot over f32 weights (its F32 and block branches): x [n, dim], w [n_out, dim]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, dim = x.shape
    assert w.shape[1] == dim
    out = np.zeros((n, w.shape[0]), dtype=np.float32)
    lib().or_project_f32(x, n, dim, w, w.shape[0], out)
    return out


def attn_proj(attn: np.ndarray, wo_bits: np.ndarray, act: np.ndarray):
    """main_attn_proj: returns (act + dot, dot) for attn [n, attn_dim] f32, wo [dim, attn_dim]
    f16 bits, act [n, dim] f32 (not modified)."""
    attn = np.ascontiguousarray(attn, dtype=np.float32)
    wo_bits = np.ascontiguousarray(wo_bits, dtype=np.uint16)
    out = np.ascontiguousarray(act, dtype=np.float32).copy()
    n, attn_dim = attn.shape
    dim = wo_bits.shape[0]
    stash = np.zeros((n, dim), np.float32)
    lib().or_attn_proj(attn, n, attn_dim, wo_bits, dim, out, stash.ctypes.data)
    return out, stash


def qk_norm_row(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """apply_qk_norm (attention.rs:92-108) of one head vector through the C oracle."""
    out = np.ascontiguousarray(x, np.float32).copy()
    lib().or_qk_norm_row(out, out.size, np.ascontiguousarray(w, np.float32), float(eps))
    return out


def rope_table(n_pos: int, rope_dim: int, base: float, scale: float = 1.0,
               yarn_alpha: float = 0.0, yarn_beta: float = 0.0) -> np.ndarray:
    """[n_pos, rope_dim/2, 2] (cos, sin) table, preflight.rs:71-111 (YaRN when scale < 1 and
    0 < yarn_alpha < yarn_beta, linear otherwise)."""
    t = np.zeros((n_pos, rope_dim // 2, 2), np.float32)
    rc = lib().or_rope_table_yarn(t, n_pos, rope_dim, base, scale, yarn_alpha, yarn_beta)
    if rc != 0:
        raise ValueError("unsupported rope parameters")
    return t


def rope_rotate(x: np.ndarray, table_row: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().or_rope_rotate(y, table_row.shape[0] * 2, np.ascontiguousarray(table_row, np.float32))
    return y


def quantize_row(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    assert x.ndim == 1 and x.size % 8 == 0
    words = np.zeros(x.size // 8, np.uint32)
    s = ctypes.c_float()
    lib().or_quantize_row(x, x.size, ctypes.byref(s), words)
    return np.float32(s.value), words


def dequantize_row(words: np.ndarray, scale) -> np.ndarray:
    words = np.ascontiguousarray(words, np.uint32)
    out = np.zeros(words.size * 8, np.float32)
    lib().or_dequantize_row(words, out.size, float(np.float32(scale)), out)
    return out


class OracleKV:
    """Per-sequence INT4 caches in the reference layout, driven like the reference
    KvCache (src/runtime/kvcache.rs): append at the current length, then advance."""

    def __init__(self, n_seq, max_seq, n_kv, hd, rope_table_arr):
        self.n_seq, self.max_seq, self.n_kv, self.hd = n_seq, max_seq, n_kv, hd
        self.k_packed = np.zeros((n_seq, max_seq, n_kv, hd // 8), np.uint32)
        self.v_packed = np.zeros_like(self.k_packed)
        self.k_scale = np.zeros((n_seq, max_seq, n_kv), np.float32)
        self.v_scale = np.zeros_like(self.k_scale)
        self.table = np.ascontiguousarray(rope_table_arr, np.float32)
        self.rope_dim = self.table.shape[1] * 2
        self.lens = np.zeros(n_seq, np.int32)
        # sliding-window compaction state (kv_cache.rs:41-46): window base and sink count
        self.rot = np.zeros(n_seq, np.int32)
        self.n_sink = np.zeros(n_seq, np.int32)
        # Qwen3 QK norm (attention.rs:92-108, :186-189): per-dim weights or None, eps 1e-6
        self.q_norm = None
        self.k_norm = None
        self.norm_eps = 1e-6

    def append(self, k: np.ndarray, v: np.ndarray):
        """k, v: [n_seq, n_tok, n_kv, hd] raw f32; written at each sequence's length."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        n_tok = k.shape[1]
        assert (self.lens + n_tok <= self.max_seq).all()
        assert (self.lens + self.rot + n_tok <= self.table.shape[0]).all()
        lib().or_append_batch(self.k_packed, self.v_packed, self.k_scale, self.v_scale,
                              self.n_seq, self.max_seq, self.n_kv, self.hd, self.rope_dim,
                              self.table, k, v, self.lens, n_tok, self.rot, self.n_sink,
                              self._w(self.k_norm), float(self.norm_eps))

    def attend(self, q: np.ndarray, n_tok: int, softcap: float = 0.0, threads: int = 1):
        """q: [n_seq, n_tok, n_head, hd] raw f32 for the n_tok tokens just appended (query
        positions lens[s]..lens[s]+n_tok-1).  Returns out of the same shape."""
        q = np.ascontiguousarray(q, np.float32)
        n_head = q.shape[2]
        out = np.zeros_like(q)
        lib().or_attend_batch(self.k_packed, self.v_packed, self.k_scale, self.v_scale,
                              self.n_seq, self.max_seq, n_head, self.n_kv, self.hd,
                              self.rope_dim, self.table, q, self.lens, n_tok, float(softcap),
                              out, int(threads), self.rot, self._w(self.q_norm),
                              float(self.norm_eps))
        return out

    def attend_one(self, q_seq: np.ndarray, seq: int, head: int, softcap: float = 0.0):
        """One (sequence, head): q_seq [n_tok, n_head, hd] for the tokens just appended to
        `seq`.  Returns [n_tok, hd]."""
        q_seq = np.ascontiguousarray(q_seq, np.float32)
        n_tok, n_head, hd = q_seq.shape
        out = np.zeros_like(q_seq)
        lib().or_attend_one(self.k_packed, self.v_packed, self.k_scale, self.v_scale,
                            self.max_seq, n_head, self.n_kv, self.hd, self.rope_dim, self.table,
                            q_seq, int(self.lens[seq]), n_tok, seq, head, float(softcap), out,
                            int(self.rot[seq]), self._w(self.q_norm), float(self.norm_eps))
        return out[:, head]

    def _w(self, w):
        """Norm weights as a C pointer (None: no norm); the array is kept alive on self."""
        if w is None:
            return None
        w = np.ascontiguousarray(w, np.float32)
        assert w.shape == (self.hd,)
        self._keep = getattr(self, "_keep", []) + [w]
        self._keep = self._keep[-4:]
        return w.ctypes.data

    def advance(self, n_tok: int):
        """complete_decode / complete_prefill: lengths advance after all layers."""
        self.lens += n_tok

    def shift(self, seq: int, keep_sink: int, shift_amt: int):
        """RopeShiftPipeline::execute_int4 (pipeline_shift.rs:360-566) for one sequence of this
        single-layer cache: slots keep_sink+shift_amt.. move down by shift_amt.  The caller then
        advances the window base and sets the length, as the reference's caller does."""
        lib().or_shift_seq(self.k_packed, self.v_packed, self.k_scale, self.v_scale,
                           self.max_seq, self.n_kv, self.hd, int(seq), int(keep_sink),
                           int(shift_amt), int(self.lens[seq]))
        self.n_sink[seq] = keep_sink

    def advance_window_base(self, seq: int, shift_amt: int):
        """KVCache::advance_window_base (kv_cache.rs:277-279)."""
        self.rot[seq] += shift_amt
