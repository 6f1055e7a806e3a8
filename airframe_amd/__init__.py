"""airframe_amd -- MI355X (gfx950) INT4 KV-cache path: RoPE-fused quantize-on-append, split-K
GQA decode attention and chunked-prefill attention over the INT4 cache, behind the C ABI in
include/turboshimmy.h."""
from ._lib import LIB_PATH, TsError, load  # noqa: F401

__all__ = ["LIB_PATH", "TsError", "load", "KVCache", "RopeTable"]


def __getattr__(name):
    if name in ("KVCache", "RopeTable"):
        from . import kv_cache
        return getattr(kv_cache, name)
    raise AttributeError(name)
