"""GPU test of ts_attn_decode_append_noalloc, the allocation-free variant of
ts_attn_decode_append (its split partials live in the library's per-GPU scratch array): on two
identical caches, the variant and the workspace entry point give bit-identical outputs and
cache contents, on two calls in a row (the second with smaller contexts and fewer splits), and
a call whose partials would not fit the scratch array is refused."""
import ctypes

import numpy as np
import pytest
import torch

from airframe_amd import _lib, synth
from airframe_amd._lib import load
from airframe_amd.kv_cache import KVCache, RopeTable, _stream
from tests.gpu_util import dev, say

pytestmark = pytest.mark.gpu


def _noalloc(kv, layer, k, v, q, rope, out):
    return load().ts_attn_decode_append_noalloc(
        kv.handle, layer, ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
        ctypes.c_void_p(q.data_ptr()), q.shape[1], rope.handle, ctypes.c_float(0.0),
        ctypes.c_void_p(out.data_ptr()), _stream())


def test_noalloc_matches_workspace_entry_point(gpu):
    n_seq, n_kv, hd, n_head = 4, 8, 128, 32
    max_seq = 8448
    rope = RopeTable(max_seq, hd, 1e6)
    rng = np.random.default_rng(900)
    a = KVCache.new_int4(1, n_kv, hd, max_seq, n_seq)
    b = KVCache.new_int4(1, n_kv, hd, max_seq, n_seq)
    for t0 in range(0, 8200, 2050):
        k = dev(synth.normal(rng, (n_seq, 2050, n_kv, hd)))
        v = dev(synth.normal(rng, (n_seq, 2050, n_kv, hd)))
        for c in (a, b):
            c.append_quant(0, k, v, rope)
            c.increment(2050)
    # first call: long contexts, 16 splits per sequence; second call: shorter contexts, 6
    for call, lens in enumerate(([8000, 7000, 8100, 5000], [1500, 900, 1200, 700])):
        say(f"noalloc call {call}: lens {lens}")
        for c in (a, b):
            for s, l in enumerate(lens):
                c.set_seq_len(l, seq=s)
        k = dev(synth.normal(rng, (n_seq, 1, n_kv, hd)))
        v = dev(synth.normal(rng, (n_seq, 1, n_kv, hd)))
        q = dev(synth.normal(rng, (n_seq, n_head, hd)))
        ref = a.attn_decode_append(0, k, v, q, rope)
        out = torch.full_like(q, float("nan"))
        rc = _noalloc(b, 0, k, v, q, rope, out)
        assert rc == 0, _lib.load().ts_status_string(rc)
        torch.cuda.synchronize()
        r, o = ref.cpu().numpy(), out.cpu().numpy()
        assert np.isfinite(o).all()
        assert np.array_equal(r.view(np.uint32), o.view(np.uint32)), \
            f"call {call}: max diff {np.abs(r - o).max()}"
        for s, l in enumerate(lens):
            ea, eb = a.export(0, s, l, 1), b.export(0, s, l, 1)
            for x, y in zip(ea, eb):
                assert torch.equal(x, y), f"call {call} seq {s}: appended row differs"


def test_noalloc_refuses_partials_beyond_scratch(gpu):
    """A ragged batch (one long sequence among short ones, 8 query heads per kv head) plans
    many splits for the long one, and the partials of n_seq * n_head * splits rows would
    exceed 8 MiB."""
    say("noalloc over the scratch limit")
    n_seq, n_kv, hd, n_head = 32, 8, 128, 64
    kv = KVCache.new_int4(1, n_kv, hd, 30100, n_seq)
    rope = RopeTable(30100, hd, 1e6)
    kv.set_seq_len(30000, seq=0)
    for s in range(1, n_seq):
        kv.set_seq_len(100, seq=s)
    k = torch.zeros((n_seq, 1, n_kv, hd), device="cuda")
    q = torch.zeros((n_seq, n_head, hd), device="cuda")
    out = torch.empty_like(q)
    rc = _noalloc(kv, 0, k, k, q, rope, out)
    assert rc == _lib.TS_ERR_WORKSPACE
    kv.attn_decode_append(0, k, k, q, rope, out=out)  # the workspace entry point still runs
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()
