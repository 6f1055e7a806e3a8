"""GPU parity with partial rotary embeddings (rope_dim < head_dim: only the first rope_dim/2
pairs rotate, rope.rs:180-197 with the table of preflight.rs:71-111 built for rope_dim): the
append's codes bit-exact, and fused decode, decode (both split kernels), prefill and the QKV
projection's cache writes against the oracle."""
import numpy as np
import pytest
import torch

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say
from tests.test_gpu_qkv import run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hd,rope_dim,n_seq,n_kv,n_head,ctx", [
    (128, 64, 2, 2, 8, 300),     # G = 4, short splits: the 16x16x32 decode kernel
    (128, 32, 32, 8, 32, 2100),  # G = 4, splits of >= 1024 positions: the 4x4x4 decode kernel
    (64, 32, 2, 2, 16, 300),     # hd 64, G = 8
])
def test_partial_rotary(gpu, hd, rope_dim, n_seq, n_kv, n_head, ctx):
    say(f"partial rotary hd={hd} rope_dim={rope_dim} n_seq={n_seq} n_kv={n_kv} n_head={n_head} ctx={ctx}")
    rng = np.random.default_rng(rope_dim + ctx)
    p = Pair(n_seq, n_kv, hd, ctx + 64, 1e6, rope_dim=rope_dim)
    done = 0
    while done < ctx:                      # ragged chunks through the append kernel
        m = min(777, ctx - done)
        k = synth.normal(rng, (n_seq, m, n_kv, hd))
        v = synth.normal(rng, (n_seq, m, n_kv, hd))
        p.append(k, v)
        p.advance(m)
        done += m
    p.check_codes()
    # fused append + decode
    k = synth.normal(rng, (n_seq, 1, n_kv, hd))
    v = synth.normal(rng, (n_seq, 1, n_kv, hd))
    q = synth.normal(rng, (n_seq, n_head, hd))
    out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope).cpu().numpy()
    p.ora.append(k, v)
    assert_close(out, p.ora.attend(q[:, None], 1, threads=8)[:, 0], "fused decode")
    p.advance(1)
    # prefill chunk
    k = synth.normal(rng, (n_seq, 20, n_kv, hd))
    v = synth.normal(rng, (n_seq, 20, n_kv, hd))
    q = synth.normal(rng, (n_seq, 20, n_head, hd))
    p.append(k, v)
    out = p.gpu.attn_prefill(0, dev(q), p.rope).cpu().numpy()
    assert_close(out, p.ora.attend(q, 20, threads=8), "prefill")
    p.advance(20)
    # the QKV projection writes the same codes as the append of its own projections
    run_case(p, rng, 1, 256, n_head)
    run_case(p, rng, 9, 256, n_head)
    p.check_codes()
