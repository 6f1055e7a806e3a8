"""Host-side mirror of airframe's INT4 KV-cache call surface over the C ABI.

Names follow the reference (src/backend/bindless/kv_cache.rs, pipeline/layer.rs,
preflight.rs); buffers are torch tensors on the current HIP device, used only as device
memory and streams.  Errors the reference reports as panics or ``Err`` raise ``TsError``
with the library's status code (``TS_ERR_OVERFLOW`` for ``increment`` past the window, as
kv_cache.rs:284-293 returns Err).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import KvDesc, check, load


def _stream(stream=None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t: torch.Tensor, dtype: torch.dtype, what: str) -> ctypes.c_void_p:
    if not t.is_cuda:
        raise ValueError(f"{what} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


class RopeTable:
    """PreflightResources' RoPE table (preflight.rs:71-142): host-computed cos/sin, uploaded."""

    def __init__(self, n_pos: int, rope_dim: int, base: float, scale: float = 1.0,
                 yarn_alpha: float = 0.0, yarn_beta: float = 0.0):
        """YaRN (preflight.rs:77-97) when scale < 1 and 0 < yarn_alpha < yarn_beta; n_pos is
        the table length, the spec's n_ctx."""
        L = load()
        h = ctypes.c_void_p()
        check("ts_rope_create_yarn", L.ts_rope_create_yarn(n_pos, rope_dim, base, scale, yarn_alpha, yarn_beta,
                                                            ctypes.byref(h)))
        self._h = h
        self.n_pos, self.rope_dim, self.base, self.scale = n_pos, rope_dim, base, scale

    @staticmethod
    def host_table(n_pos: int, rope_dim: int, base: float, scale: float = 1.0,
                   yarn_alpha: float = 0.0, yarn_beta: float = 0.0):
        import numpy as np
        t = np.zeros((n_pos, rope_dim // 2, 2), np.float32)
        check("ts_rope_table_host_yarn",
              load().ts_rope_table_host_yarn(t.ctypes.data_as(ctypes.c_void_p), n_pos, rope_dim, base, scale,
                                             yarn_alpha, yarn_beta))
        return t

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            load().ts_rope_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    """INT4 KV cache for ``n_seq`` independent sequences (kv_cache.rs KVCache with a batch
    dimension; each sequence behaves like one reference cache)."""

    def __init__(self, n_layers: int, n_head_kv: int, head_dim: int, max_seq_len: int,
                 n_seq: int = 1):
        L = load()
        d = KvDesc(n_layers, n_seq, n_head_kv, head_dim, max_seq_len)
        h = ctypes.c_void_p()
        check("ts_kv_create", L.ts_kv_create(ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        self.n_layers, self.n_seq, self.n_head_kv = n_layers, n_seq, n_head_kv
        self.head_dim, self.max_seq_len = head_dim, max_seq_len
        self._ws = {}
        # ts_kv_create allocates on the current device; copies out of the cache go there too
        self.device = torch.device("cuda", torch.cuda.current_device())

    @classmethod
    def new_int4(cls, n_layers, n_head_kv, head_dim, max_seq_len, n_seq=1):
        """KVCache::new_int4 (kv_cache.rs:88-96)."""
        return cls(n_layers, n_head_kv, head_dim, max_seq_len, n_seq)

    @staticmethod
    def bytes_for(n_layers, n_head_kv, head_dim, max_seq_len, n_seq=1) -> int:
        d = KvDesc(n_layers, n_seq, n_head_kv, head_dim, max_seq_len)
        b = ctypes.c_uint64()
        check("ts_kv_bytes", load().ts_kv_bytes(ctypes.byref(d), ctypes.byref(b)))
        return b.value

    @property
    def handle(self):
        return self._h

    def is_int4(self) -> bool:
        return True

    def get_seq_len(self, seq: int = 0) -> int:
        v = ctypes.c_int32()
        check("ts_kv_seq_len", load().ts_kv_seq_len(self._h, seq, ctypes.byref(v)))
        return v.value

    def seq_lens(self):
        return [self.get_seq_len(s) for s in range(self.n_seq)]

    def max_len(self) -> int:
        return self.max_seq_len

    def increment(self, n_tok: int = 1, stream=None):
        check("ts_kv_increment", load().ts_kv_increment(self._h, n_tok, _stream(stream)))

    def set_seq_len(self, new_len: int, seq: int = 0, stream=None):
        check("ts_kv_set_seq_len", load().ts_kv_set_seq_len(self._h, seq, new_len, _stream(stream)))

    def reset(self, seq: int | None = None, stream=None):
        """KVCache::reset (kv_cache.rs:256-259): length, window base and sink count to 0, for
        every sequence or only `seq`."""
        if seq is None:
            check("ts_kv_reset", load().ts_kv_reset(self._h, _stream(stream)))
        else:
            check("ts_kv_reset_seq", load().ts_kv_reset_seq(self._h, seq, _stream(stream)))

    # ---- QK norm (Qwen3: attention.rs:92-108 before RoPE, :186-189) ----------------------

    def set_qk_norm(self, layer: int, q_norm: torch.Tensor | None, k_norm: torch.Tensor | None,
                    eps: float = 1e-6):
        """Per-head RMSNorm of q and K (weights [head_dim] f32 on the device, or None) for one
        layer, applied by the append and attention calls before RoPE.  The tensors are kept
        alive by the cache."""
        for w in (q_norm, k_norm):
            if w is not None and (w.dtype != torch.float32 or w.numel() != self.head_dim or
                                  not w.is_cuda or not w.is_contiguous()):
                raise ValueError("norm weights must be contiguous f32 [head_dim] on the device")
        if not hasattr(self, "_norms"):
            self._norms = {}
        self._norms[layer] = (q_norm, k_norm)
        ptr = lambda w: ctypes.c_void_p(w.data_ptr()) if w is not None else None
        check("ts_kv_set_qk_norm",
              load().ts_kv_set_qk_norm(self._h, layer, ptr(q_norm), ptr(k_norm), eps))

    # ---- sliding-window compaction (pipeline_shift.rs, kv_cache.rs window_base) ---------

    def get_window_base(self, seq: int = 0) -> int:
        """KVCache::get_window_base (kv_cache.rs:241-243)."""
        v = ctypes.c_int32()
        check("ts_kv_window_base", load().ts_kv_window_base(self._h, seq, ctypes.byref(v)))
        return v.value

    def advance_window_base(self, shift_amt: int, seq: int = 0, stream=None):
        """KVCache::advance_window_base (kv_cache.rs:277-279)."""
        check("ts_kv_advance_window_base",
              load().ts_kv_advance_window_base(self._h, seq, shift_amt, _stream(stream)))

    def shift_int4(self, layer: int, keep_sink: int, shift_amt: int, seq: int = 0,
                   workspace: torch.Tensor = None, stream=None):
        """RopeShiftPipeline::execute_int4 (pipeline_shift.rs:360-566) for one layer of one
        sequence: slots keep_sink+shift_amt.. move down by shift_amt, sinks stay."""
        if workspace is None:
            if "shift" not in self._ws:
                b = ctypes.c_uint64()
                check("ts_kv_shift_workspace", load().ts_kv_shift_workspace(self._h, ctypes.byref(b)))
                self._ws["shift"] = torch.empty(max(b.value, 16), dtype=torch.uint8, device=self.device)
            workspace = self._ws["shift"]
        check("ts_kv_shift",
              load().ts_kv_shift(self._h, layer, seq, keep_sink, shift_amt,
                                 ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
                                 _stream(stream)))

    def compact(self, keep_sink: int, shift_amt: int, seq: int = 0, stream=None):
        """The helical-compaction sequence of the reference's caller for one sequence: every
        layer shifted, then advance_window_base and set_seq_len(len - shift_amt).  Does nothing
        when len <= keep_sink + shift_amt."""
        n = self.get_seq_len(seq)
        if n <= keep_sink + shift_amt or shift_amt == 0:
            return
        for layer in range(self.n_layers):
            self.shift_int4(layer, keep_sink, shift_amt, seq, stream=stream)
        self.advance_window_base(shift_amt, seq, stream)
        self.set_seq_len(n - shift_amt, seq, stream)

    # ---- hot path ----------------------------------------------------------------------

    def append_quant(self, layer: int, k: torch.Tensor, v: torch.Tensor, rope: RopeTable,
                     stream=None):
        """Quantize-on-append (sh_quantize_kv.wgsl, RoPE fused on K).  k, v:
        [n_seq, n_tok, n_head_kv, head_dim] f32 on the device."""
        n_tok = k.shape[1]
        self._check_kv(k, v, n_tok)
        check("ts_append_quant",
              load().ts_append_quant(self._h, layer, _ptr(k, torch.float32, "k"),
                                     _ptr(v, torch.float32, "v"), n_tok, rope.handle,
                                     _stream(stream)))

    def requantize_all_kv_int4(self, layer: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                               seq_len: int, rope: RopeTable | None = None, stream=None):
        """requantize_all_kv_int4 (layer.rs:1161-1246) for one layer from f32 caches
        [n_seq, ld_pos, n_head_kv, head_dim]."""
        if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != self.n_seq:
            raise ValueError("k_cache/v_cache must be [n_seq, ld_pos, n_head_kv, head_dim]")
        check("ts_requant_all",
              load().ts_requant_all(self._h, layer, _ptr(k_cache, torch.float32, "k_cache"),
                                    _ptr(v_cache, torch.float32, "v_cache"), seq_len,
                                    k_cache.shape[1], rope.handle if rope else None,
                                    _stream(stream)))

    def workspace(self, n_head: int) -> torch.Tensor:
        if n_head not in self._ws:
            b = ctypes.c_uint64()
            check("ts_attn_decode_workspace",
                  load().ts_attn_decode_workspace(self._h, n_head, ctypes.byref(b)))
            self._ws[n_head] = torch.empty(max(b.value, 4), dtype=torch.uint8, device=self.device)
        return self._ws[n_head]

    def attn_decode(self, layer: int, q: torch.Tensor, rope: RopeTable, out: torch.Tensor = None,
                    softcap: float = 0.0, workspace: torch.Tensor = None, stream=None):
        """INT4 decode attention (main_attn_out_int4's role).  q: [n_seq, n_head, head_dim]."""
        n_head = q.shape[1]
        if q.dim() != 3 or q.shape[0] != self.n_seq or q.shape[2] != self.head_dim:
            raise ValueError("q must be [n_seq, n_head, head_dim]")
        out = self._out_like(q, out)
        ws = workspace if workspace is not None else self.workspace(n_head)
        check("ts_attn_decode",
              load().ts_attn_decode(self._h, layer, _ptr(q, torch.float32, "q"), n_head,
                                    rope.handle, softcap, _ptr(out, torch.float32, "out"),
                                    ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
        return out

    def attn_decode_append(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
                           rope: RopeTable, out: torch.Tensor = None, softcap: float = 0.0,
                           workspace: torch.Tensor = None, stream=None, advance: bool = False):
        """append_quant(layer, k, v) + attn_decode(layer, q) in one launch (the quantize_kv +
        main_attn_out_int4 pair of run_layer_with_cache_int4).  k, v: [n_seq, 1, n_head_kv,
        head_dim] or [n_seq, n_head_kv, head_dim]; q: [n_seq, n_head, head_dim].
        advance=True (the step's last layer): every length then advances by one, as
        increment(1) would, inside the same launch (ts_attn_decode_append_advance)."""
        n_head = q.shape[1]
        if q.dim() != 3 or q.shape[0] != self.n_seq or q.shape[2] != self.head_dim:
            raise ValueError("q must be [n_seq, n_head, head_dim]")
        self._check_kv(k.reshape(self.n_seq, 1, self.n_head_kv, self.head_dim),
                       v.reshape(self.n_seq, 1, self.n_head_kv, self.head_dim), 1)
        out = self._out_like(q, out)
        ws = workspace if workspace is not None else self.workspace(n_head)
        fn = "ts_attn_decode_append_advance" if advance else "ts_attn_decode_append"
        check(fn,
              getattr(load(), fn)(self._h, layer, _ptr(k, torch.float32, "k"),
                                           _ptr(v, torch.float32, "v"), _ptr(q, torch.float32, "q"),
                                           n_head, rope.handle, softcap,
                                           _ptr(out, torch.float32, "out"),
                                           ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                           _stream(stream)))
        return out

    def attn_prefill(self, layer: int, q: torch.Tensor, rope: RopeTable, out: torch.Tensor = None,
                     softcap: float = 0.0, stream=None):
        """Chunked-prefill causal attention.  q: [n_seq, n_tok, n_head, head_dim]."""
        if q.dim() != 4 or q.shape[0] != self.n_seq or q.shape[3] != self.head_dim:
            raise ValueError("q must be [n_seq, n_tok, n_head, head_dim]")
        out = self._out_like(q, out)
        check("ts_attn_prefill",
              load().ts_attn_prefill(self._h, layer, _ptr(q, torch.float32, "q"), q.shape[2],
                                     q.shape[1], rope.handle, softcap,
                                     _ptr(out, torch.float32, "out"), _stream(stream)))
        return out

    def export(self, layer: int, seq: int, pos0: int, n_pos: int, stream=None):
        """Packed K/V and scales of positions [pos0, pos0+n_pos) in the reference layout
        ([pos][n_head_kv][head_dim/8] u32 as int32 bits, [pos][n_head_kv] f32), on the
        cache's device."""
        dev = self.device
        kp = torch.empty((n_pos, self.n_head_kv, self.head_dim // 8), dtype=torch.int32, device=dev)
        vp = torch.empty_like(kp)
        ks = torch.empty((n_pos, self.n_head_kv), dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        check("ts_kv_export",
              load().ts_kv_export(self._h, layer, seq, pos0, n_pos, ctypes.c_void_p(kp.data_ptr()),
                                  ctypes.c_void_p(vp.data_ptr()), ctypes.c_void_p(ks.data_ptr()),
                                  ctypes.c_void_p(vs.data_ptr()), _stream(stream)))
        return kp, vp, ks, vs

    # The reference's per-layer buffer getters (kv_cache.rs:312-345).  The reference hands out
    # its buffers; this cache keeps its own tiled layout, so these return copies of one
    # sequence's whole layer (max_seq_len positions) in the reference layout, through export.
    # Each single getter runs one export of all four arrays and keeps one; a caller that wants
    # several of them takes get_buffers, which moves the bytes once.
    def get_buffers(self, layer: int, seq: int = 0):
        """(k_packed, v_packed, k_scale, v_scale) of one sequence's layer, one export."""
        return self.export(layer, seq, 0, self.max_seq_len)

    def get_k_packed_buffer(self, layer: int, seq: int = 0) -> torch.Tensor:
        return self.get_buffers(layer, seq)[0]

    def get_v_packed_buffer(self, layer: int, seq: int = 0) -> torch.Tensor:
        return self.get_buffers(layer, seq)[1]

    def get_k_scale_buffer(self, layer: int, seq: int = 0) -> torch.Tensor:
        return self.get_buffers(layer, seq)[2]

    def get_v_scale_buffer(self, layer: int, seq: int = 0) -> torch.Tensor:
        return self.get_buffers(layer, seq)[3]

    def calculate_offset(self, pos: int, head: int, dim: int) -> int:
        """Byte offset of (pos, head, dim) in the reference's f32 staging layout
        [pos][n_head_kv][head_dim] (kv_cache.rs:366-369)."""
        return ((pos * self.n_head_kv + head) * self.head_dim + dim) * 4

    def qkv_workspace(self, dim: int, n_tok: int, n_head: int) -> torch.Tensor:
        key = ("qkv", dim, n_tok, n_head)
        if key not in self._ws:
            b = ctypes.c_uint64()
            check("ts_qkv_workspace",
                  load().ts_qkv_workspace(self._h, dim, n_tok, n_head, ctypes.byref(b)))
            self._ws[key] = torch.empty(max(b.value, 16), dtype=torch.uint8, device=self.device)
        return self._ws[key]

    def qkv_append(self, layer: int, x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor,
                   wv: torch.Tensor, rope: RopeTable, q_out: torch.Tensor = None,
                   kv_out: tuple | None = None, workspace: torch.Tensor = None, stream=None,
                   planes: int = 1):
        """main_qkv + quantize_kv in one pass: q = Wq x (returned), k = Wk x and v = Wv x
        quantized into the cache at len[s] + t.  x: [n_seq, n_tok, dim] f32; wq: [n_head *
        head_dim, dim], wk, wv: [n_head_kv * head_dim, dim] f16.  kv_out: optional (k, v)
        tensors [n_seq, n_tok, n_head_kv, head_dim] f32 that receive the raw projections.
        planes=2: weight rows of [hi dim | lo dim] f16 (weights.to_f16x2, the F32 and GGUF block
        formats at about f32 accuracy) through ts_qkv_append_x2."""
        if x.dim() != 3 or x.shape[0] != self.n_seq:
            raise ValueError("x must be [n_seq, n_tok, dim]")
        n_tok, dim = x.shape[1], x.shape[2]
        n_head = wq.shape[0] // self.head_dim
        kv_rows = self.n_head_kv * self.head_dim
        if planes not in (1, 2):
            raise ValueError("planes must be 1 or 2")
        wd = planes * dim
        if (wq.shape != (n_head * self.head_dim, wd) or wk.shape != (kv_rows, wd)
                or wv.shape != (kv_rows, wd)):
            raise ValueError("wq must be [n_head*head_dim, planes*dim], wk/wv [n_head_kv*head_dim, planes*dim]")
        want = (self.n_seq, n_tok, n_head, self.head_dim)
        if q_out is None:
            q_out = torch.empty(want, dtype=torch.float32, device=x.device)
        elif tuple(q_out.shape) != want:
            raise ValueError(f"q_out must be {want}")
        kp = vp = None
        if kv_out is not None:
            k_out, v_out = kv_out
            self._check_kv(k_out, v_out, n_tok)
            kp, vp = _ptr(k_out, torch.float32, "k_out"), _ptr(v_out, torch.float32, "v_out")
        ws = workspace if workspace is not None else self.qkv_workspace(dim, n_tok, n_head)
        fn = "ts_qkv_append" if planes == 1 else "ts_qkv_append_x2"
        check(fn,
              getattr(load(), fn)(self._h, layer, _ptr(x, torch.float32, "x"), dim, n_tok,
                                   _ptr(wq, torch.float16, "wq"), _ptr(wk, torch.float16, "wk"),
                                   _ptr(wv, torch.float16, "wv"), n_head, rope.handle,
                                   _ptr(q_out, torch.float32, "q_out"), kp, vp,
                                   ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
        return q_out

    def qkv_append_gguf(self, layer: int, x: torch.Tensor, ggml_type: int, wq: torch.Tensor,
                        wk: torch.Tensor, wv: torch.Tensor, rope: RopeTable,
                        q_out: torch.Tensor = None, kv_out: tuple | None = None,
                        workspace: torch.Tensor = None, stream=None):
        """qkv_append with the weights as the GGUF blob's Q4_K / Q5_K / Q8_0 / Q4_0 / Q5_0 blocks
        (uint8 CUDA tensors of [rows, the row's block bytes] or flat), read inside the projection loop
        (ts_qkv_append_gguf).  dim a multiple of 256."""
        if x.dim() != 3 or x.shape[0] != self.n_seq:
            raise ValueError("x must be [n_seq, n_tok, dim]")
        n_tok, dim = x.shape[1], x.shape[2]
        n_head = q_out.shape[2] if q_out is not None else None
        from .weights import src_bytes
        row_bytes = src_bytes(ggml_type, 1, dim)
        if n_head is None:
            n_head = wq.numel() // (row_bytes * self.head_dim)
        kv_rows = self.n_head_kv * self.head_dim
        for name, wt, rows in (("wq", wq, n_head * self.head_dim), ("wk", wk, kv_rows), ("wv", wv, kv_rows)):
            if wt.dtype != torch.uint8 or wt.numel() != rows * row_bytes:
                raise ValueError(f"{name} must hold {rows} rows of {row_bytes} GGUF bytes (uint8)")
        want = (self.n_seq, n_tok, n_head, self.head_dim)
        if q_out is None:
            q_out = torch.empty(want, dtype=torch.float32, device=x.device)
        elif tuple(q_out.shape) != want:
            raise ValueError(f"q_out must be {want}")
        kp = vp = None
        if kv_out is not None:
            k_out, v_out = kv_out
            self._check_kv(k_out, v_out, n_tok)
            kp, vp = _ptr(k_out, torch.float32, "k_out"), _ptr(v_out, torch.float32, "v_out")
        ws = workspace
        if ws is None:
            key = ("qkv_gguf", ggml_type, dim, n_tok, n_head)
            if key not in self._ws:
                b = ctypes.c_uint64()
                check("ts_qkv_gguf_workspace",
                      load().ts_qkv_gguf_workspace(self._h, ggml_type, dim, n_tok, n_head, ctypes.byref(b)))
                self._ws[key] = torch.empty(max(b.value, 16), dtype=torch.uint8, device=self.device)
            ws = self._ws[key]
        check("ts_qkv_append_gguf",
              load().ts_qkv_append_gguf(self._h, layer, _ptr(x, torch.float32, "x"), dim, n_tok, ggml_type,
                                        _ptr(wq, torch.uint8, "wq"), _ptr(wk, torch.uint8, "wk"),
                                        _ptr(wv, torch.uint8, "wv"), n_head, rope.handle,
                                        _ptr(q_out, torch.float32, "q_out"), kp, vp,
                                        ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
        return q_out

    @staticmethod
    def _out_like(q, out):
        """A caller's output tensor must have q's shape (the kernels write that many floats)."""
        if out is None:
            return torch.empty_like(q)
        if tuple(out.shape) != tuple(q.shape):
            raise ValueError(f"out must have q's shape {tuple(q.shape)}, got {tuple(out.shape)}")
        return out

    def _check_kv(self, k, v, n_tok):
        want = (self.n_seq, n_tok, self.n_head_kv, self.head_dim)
        if tuple(k.shape) != want or tuple(v.shape) != want:
            raise ValueError(f"k/v must be {want}")

    def close(self):
        if self._h:
            load().ts_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# keep the status codes reachable from the package
TS_ERR_OVERFLOW = _lib.TS_ERR_OVERFLOW


_proj_ws: dict = {}


def attn_out_proj(attn: torch.Tensor, wo: torch.Tensor, act: torch.Tensor,
                  stash: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                  stream=None, planes: int = 1) -> torch.Tensor:
    """main_attn_proj (sh_layer_v1.wgsl:763-821, F16 weights): act += Wo attn per token, the raw
    product into `stash` when given.  attn: [n_tok, attn_dim] f32 (any leading shape flattened
    to tokens), wo: [dim, attn_dim] f16, act (and stash): [n_tok, dim] f32.  Returns act.
    planes=2: wo rows of [hi attn_dim | lo attn_dim] (weights.to_f16x2), ts_attn_out_proj_x2."""
    attn2 = attn.reshape(-1, attn.shape[-1])
    n_tok, attn_dim = attn2.shape
    dim = wo.shape[0]
    if planes not in (1, 2) or wo.shape != (dim, planes * attn_dim):
        raise ValueError("wo must be [dim, planes*attn_dim], planes 1 or 2")
    if act.numel() != n_tok * dim or (stash is not None and stash.numel() != n_tok * dim):
        raise ValueError("act/stash must hold [n_tok, dim]")
    ws = workspace
    if ws is None:
        key = (attn.device.index, n_tok, attn_dim, dim)
        if key not in _proj_ws:
            b = ctypes.c_uint64()
            check("ts_attn_out_proj_workspace",
                  load().ts_attn_out_proj_workspace(n_tok, attn_dim, dim, ctypes.byref(b)))
            _proj_ws[key] = torch.empty(max(b.value, 16), dtype=torch.uint8, device=attn.device)
        ws = _proj_ws[key]
    fn = "ts_attn_out_proj" if planes == 1 else "ts_attn_out_proj_x2"
    check(fn,
          getattr(load(), fn)(_ptr(attn2, torch.float32, "attn"), n_tok, attn_dim,
                                  _ptr(wo, torch.float16, "wo"), dim, _ptr(act, torch.float32, "act"),
                                  _ptr(stash, torch.float32, "stash") if stash is not None else None,
                                  ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
    return act


def attn_out_proj_gguf(attn: torch.Tensor, ggml_type: int, wo: torch.Tensor, dim: int, act: torch.Tensor,
                       stash: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                       stream=None) -> torch.Tensor:
    """attn_out_proj with wo as the GGUF blob's Q4_K / Q5_K / Q8_0 / Q4_0 / Q5_0 blocks ([dim] rows of
    attn_dim elements, uint8), read inside the projection loop (ts_attn_out_proj_gguf).  Returns
    act."""
    from .weights import src_bytes
    attn2 = attn.reshape(-1, attn.shape[-1])
    n_tok, attn_dim = attn2.shape
    if wo.dtype != torch.uint8 or wo.numel() != src_bytes(ggml_type, dim, attn_dim):
        raise ValueError("wo must hold dim rows of attn_dim / 256 GGUF blocks (uint8)")
    if act.numel() != n_tok * dim or (stash is not None and stash.numel() != n_tok * dim):
        raise ValueError("act/stash must hold [n_tok, dim]")
    ws = workspace
    if ws is None:
        key = ("gguf", ggml_type, attn.device.index, n_tok, attn_dim, dim)
        if key not in _proj_ws:
            b = ctypes.c_uint64()
            check("ts_attn_out_proj_gguf_workspace",
                  load().ts_attn_out_proj_gguf_workspace(ggml_type, n_tok, attn_dim, dim, ctypes.byref(b)))
            _proj_ws[key] = torch.empty(max(b.value, 16), dtype=torch.uint8, device=attn.device)
        ws = _proj_ws[key]
    check("ts_attn_out_proj_gguf",
          load().ts_attn_out_proj_gguf(_ptr(attn2, torch.float32, "attn"), n_tok, attn_dim, ggml_type,
                                       _ptr(wo, torch.uint8, "wo"), dim, _ptr(act, torch.float32, "act"),
                                       _ptr(stash, torch.float32, "stash") if stash is not None else None,
                                       ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
    return act
