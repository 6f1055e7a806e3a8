"""GPU parity of the fused append + decode launch (ts_attn_decode_append): the cache holds the
same codes and scales as after ts_append_quant (bit-exact against the oracle) and the outputs
match the oracle's attention over the dequantized cache, |err| <= 2e-3 + 1e-3*|ref|."""
import numpy as np
import pytest
import torch

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu


def fused_step(p: Pair, rng, n_head, scale_kv=None, scale_q=None, softcap=0.0):
    n_seq, n_kv, hd = p.n_seq, p.n_kv, p.hd
    k = synth.normal(rng, (n_seq, 1, n_kv, hd), scale_kv)
    v = synth.normal(rng, (n_seq, 1, n_kv, hd), scale_kv)
    q = synth.normal(rng, (n_seq, n_head, hd), scale_q)
    out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope, softcap=softcap).cpu().numpy()
    p.ora.append(k, v)
    ref = p.ora.attend(q[:, None], 1, softcap=softcap, threads=8)[:, 0]
    p.advance(1)
    return out, ref


def fill(p: Pair, rng, n, scale_kv=None, step=512):
    done = 0
    while done < n:
        m = min(step, n - done)
        k = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd), scale_kv)
        v = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd), scale_kv)
        p.append(k, v)
        p.advance(m)
        done += m


def test_ragged_split_edges_multistep(gpu):
    """Lengths that put the new token first, last and alone in a split, and an empty cache;
    three steps; codes of every position bit-exact afterwards."""
    say("fused ragged")
    rng = np.random.default_rng(101)
    lens = [0, 1, 31, 32, 63, 64, 255, 256, 257, 511, 512, 1023, 1024, 1500, 2046, 2047]
    p = Pair(len(lens), 2, 128, 2100, 1e6)
    fill(p, rng, max(lens))
    p.set_lens(lens)
    for _ in range(3):
        out, ref = fused_step(p, rng, 8)
        assert_close(out, ref, "fused ragged out")
    p.check_codes()


def test_qwen3_shape_outliers(gpu):
    say("fused outliers")
    rng = np.random.default_rng(102)
    n_kv, n_head, hd = 8, 32, 128
    dims = synth.outlier_dims(n_kv, hd, 5)
    skv = synth.channel_scale(n_kv, n_kv, hd, dims)
    sq = synth.channel_scale(n_head, n_kv, hd, dims)
    p = Pair(4, n_kv, hd, 3100, 1e6)
    fill(p, rng, 3000, skv[None, None])
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head, skv[None, None], sq[None])
        assert_close(out, ref, "fused outlier out")
    p.check_codes()


@pytest.mark.parametrize("n_kv,n_head,hd,softcap", [(8, 32, 64, 0.0), (2, 16, 128, 0.0), (4, 16, 64, 5.0)])
def test_shapes_and_softcap(gpu, n_kv, n_head, hd, softcap):
    say(f"fused n_kv={n_kv} n_head={n_head} hd={hd} softcap={softcap}")
    rng = np.random.default_rng(103)
    scale = np.float32(3.0) if softcap else None
    p = Pair(2, n_kv, hd, 700, 500000.0)
    fill(p, rng, 600, scale)
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head, scale, scale, softcap=softcap)
        assert_close(out, ref, "fused out")
    p.check_codes()


def test_fused_equals_separate_calls(gpu):
    """Same inputs through append_quant + attn_decode and through the fused launch: identical
    cache contents, outputs equal to within the tolerance."""
    say("fused vs separate")
    rng = np.random.default_rng(104)
    a = Pair(3, 8, 128, 1200, 1e6)
    b = Pair(3, 8, 128, 1200, 1e6)
    for t0 in range(0, 1000, 500):
        k = synth.normal(rng, (3, 500, 8, 128))
        v = synth.normal(rng, (3, 500, 8, 128))
        for p in (a, b):
            p.append(k, v)
            p.advance(500)
    k = dev(synth.normal(rng, (3, 1, 8, 128)))
    v = dev(synth.normal(rng, (3, 1, 8, 128)))
    q = dev(synth.normal(rng, (3, 32, 128)))
    a.gpu.append_quant(0, k, v, a.rope)
    oa = a.gpu.attn_decode(0, q, a.rope).cpu().numpy()
    ob = b.gpu.attn_decode_append(0, k, v, q, b.rope).cpu().numpy()
    assert_close(ob, oa, "fused vs separate")
    torch.cuda.synchronize()
    for s in range(3):
        for x, y in zip(a.gpu.export(0, s, 0, 1001), b.gpu.export(0, s, 0, 1001)):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32))


@pytest.mark.parametrize("n_head,softcap", [(32, 0.0), (24, 0.0), (8, 30.0)])
def test_long_splits(gpu, n_head, softcap):
    """Shapes whose splits are long enough (>= 4 windows per wave) for the 4x4x4 QK kernel:
    16 sequences x 8 kv heads at up to 8200 positions (split length 1088), ragged lengths on
    and around the split edges, outlier channels, G = 4, 3 and 1."""
    say(f"fused long splits n_head={n_head} softcap={softcap}")
    rng = np.random.default_rng(103 + n_head)
    n_kv, hd = 8, 128
    dims = synth.outlier_dims(n_kv, hd, 7)
    skv = synth.channel_scale(n_kv, n_kv, hd, dims)
    sq = synth.channel_scale(n_head, n_kv, hd, dims)
    lens = [8199, 8198, 4351, 1087, 1088, 1089, 2176, 3263, 5440, 6527, 7614, 100, 0, 2000, 4000, 6000]
    p = Pair(len(lens), n_kv, hd, 8210, 1e6)
    fill(p, rng, max(lens), skv[None, None], step=2048)
    p.set_lens(lens)
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head, skv[None, None], sq[None], softcap=softcap)
        assert_close(out, ref, "fused long-split out")
    p.check_codes()


def test_many_sequences(gpu):
    """300 sequences (more than one workgroup per CU on the sequence axis alone) with ragged
    short contexts: fused decode, then a prefill chunk, against the oracle; codes bit-exact."""
    say("decode/prefill with 300 sequences")
    rng = np.random.default_rng(300)
    n_seq, n_kv, n_head, hd = 300, 2, 8, 128
    p = Pair(n_seq, n_kv, hd, 160, 1e6)
    p.set_lens(rng.integers(0, 90, size=n_seq).astype(np.int32))
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head)
        assert_close(out, ref, "fused decode, 300 sequences")
    k = synth.normal(rng, (n_seq, 9, n_kv, hd))
    v = synth.normal(rng, (n_seq, 9, n_kv, hd))
    q = synth.normal(rng, (n_seq, 9, n_head, hd))
    p.append(k, v)
    out = p.gpu.attn_prefill(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q, 9, threads=8)
    assert_close(out, ref, "prefill, 300 sequences")
    p.advance(9)
    p.check_codes()
