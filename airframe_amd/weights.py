"""Projection weights in the reference's GGUF formats (main_qkv / main_attn_proj read F32, F16
and the block formats, sh_layer_v1_int4.wgsl:497-520), converted on the device into the f16
rows that KVCache.qkv_append and attn_out_proj take, through ts_weights_to_f16."""
import ctypes

from ._lib import check, load

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14


def src_bytes(ggml_type: int, n_rows: int, n_cols: int) -> int:
    """Bytes of an [n_rows][n_cols] weight matrix of that GGML type."""
    b = ctypes.c_uint64()
    check("ts_weights_src_bytes", load().ts_weights_src_bytes(ggml_type, n_rows, n_cols, ctypes.byref(b)))
    return b.value


def to_f16(ggml_type: int, src, n_rows: int, n_cols: int, stream=None, planes: int = 1):
    """src: a uint8 CUDA tensor holding the GGUF bytes of the matrix; returns [n_rows, n_cols]
    f16 on the same device (the reference's dequantized values rounded to f16), or with
    planes=2 [n_rows, 2 n_cols]: each row the values rounded to f16, then the rest rounded to
    f16 (for qkv_append / attn_out_proj with planes=2)."""
    import torch
    from .kv_cache import _stream
    need = src_bytes(ggml_type, n_rows, n_cols)
    if src.dtype != torch.uint8 or not src.is_cuda or not src.is_contiguous() or src.numel() < need:
        raise ValueError(f"src must be a contiguous uint8 CUDA tensor of at least {need} bytes")
    if planes not in (1, 2):
        raise ValueError("planes must be 1 or 2")
    out = torch.empty((n_rows, planes * n_cols), dtype=torch.float16, device=src.device)
    fn = "ts_weights_to_f16" if planes == 1 else "ts_weights_to_f16x2"
    check(fn, getattr(load(), fn)(ggml_type, ctypes.c_void_p(src.data_ptr()), n_rows, n_cols,
                                  ctypes.c_void_p(out.data_ptr()), _stream(stream)))
    return out
