"""GPU parity of the chunked-prefill attention over the INT4 cache (causal, queries at
len..len+n_tok-1) against the CPU oracle, within |err| <= 2e-3 + 1e-3*|ref|."""
import os

import numpy as np
import pytest
import torch

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu


def run_chunks(p: Pair, rng, n_head, chunks, scale_kv=None, scale_q=None, check_heads=None,
               softcap=0.0):
    for n in chunks:
        k = synth.normal(rng, (p.n_seq, n, p.n_kv, p.hd), scale_kv)
        v = synth.normal(rng, (p.n_seq, n, p.n_kv, p.hd), scale_kv)
        q = synth.normal(rng, (p.n_seq, n, n_head, p.hd), scale_q)
        p.append(k, v)
        out = p.gpu.attn_prefill(0, dev(q), p.rope, softcap=softcap).cpu().numpy()
        if check_heads is None:
            ref = p.ora.attend(q, n, softcap=softcap, threads=min(16, os.cpu_count() or 1))
            assert_close(out, ref, f"prefill chunk {n} at {p.ora.lens.tolist()}")
        else:
            for s, h in check_heads:
                ref = p.ora.attend_one(q[s], s, h, softcap=softcap)
                assert_close(out[s, :, h], ref, f"prefill seq {s} head {h} chunk at {p.ora.lens[s]}")
        p.advance(n)


def test_chunks_qwen3_4b_shape_small(gpu):
    """Config 5's head shape (32/8, hd 128) with batch 2 and 3 chunks of 96, 128 and 40."""
    say("prefill small")
    rng = np.random.default_rng(50)
    p = Pair(2, 8, 128, 300, 1e6)
    run_chunks(p, rng, 32, [96, 128, 40])
    p.check_codes()


@pytest.mark.parametrize("n_kv,n_head,hd", [(8, 24, 128), (2, 16, 64), (4, 4, 128)])
def test_chunks_group_sizes(gpu, n_kv, n_head, hd):
    say(f"prefill groups {n_kv}/{n_head}/{hd}")
    rng = np.random.default_rng(51)
    p = Pair(2, n_kv, hd, 200, 500000.0)
    p.set_lens([0, 13])
    run_chunks(p, rng, n_head, [33, 70])


def test_single_token_prefill_equals_decode(gpu):
    say("prefill n_tok=1 vs decode")
    rng = np.random.default_rng(52)
    p = Pair(3, 8, 128, 600, 1e6)
    run_chunks(p, rng, 32, [517])
    k = synth.normal(rng, (3, 1, 8, 128))
    p.append(k, k)
    q = synth.normal(rng, (3, 32, 128))
    a = p.gpu.attn_decode(0, dev(q), p.rope).cpu().numpy()
    b = p.gpu.attn_prefill(0, dev(q[:, None]), p.rope).cpu().numpy()[:, 0]
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    assert_close(a, ref, "decode")
    assert_close(b, ref, "prefill(1)")


def test_softcap_prefill(gpu):
    say("prefill softcap")
    rng = np.random.default_rng(53)
    p = Pair(1, 4, 64, 128, 10000.0)
    run_chunks(p, rng, 8, [64, 50], np.float32(3.0), np.float32(3.0), softcap=4.0)


def test_full_size_config5(gpu):
    """Config 5 at full size: Qwen3-4B shape, batch 4, 4 chunks of 512 with fused-RoPE append,
    then causal attention; the oracle checks every (sequence, token, head) output per chunk."""
    say("prefill full cfg5")
    rng = np.random.default_rng(55)
    p = Pair(4, 8, 128, 2048, 1e6)
    run_chunks(p, rng, 32, [512] * 4)
    p.check_codes()
    torch.cuda.synchronize()


def test_outlier_channels(gpu):
    """x8 outlier channels on 2% of dims in q, k and v (the shape of config 3's data): peaked
    softmax rows and large V values, where the precision of P matters."""
    say("prefill outliers")
    rng = np.random.default_rng(53)
    n_kv, n_head, hd = 8, 32, 128
    dims = synth.outlier_dims(n_kv, hd, 7)
    skv = synth.channel_scale(n_kv, n_kv, hd, dims)
    sq = synth.channel_scale(n_head, n_kv, hd, dims)
    p = Pair(2, n_kv, hd, 700, 1e6)
    run_chunks(p, rng, n_head, [256, 300, 100], skv[None, None], sq[None, None])
    p.check_codes()
