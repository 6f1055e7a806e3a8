"""GPU parity of the RoPE-fused quantize-on-append: INT4 codes and scales bit-exact with the
CPU oracle (cpu_quantize of test_int4_parity.rs:56-75 after rope.rs rotation)."""
import json
import os

import numpy as np
import pytest
import torch

from airframe_amd import TsError
from airframe_amd import _lib
from tests.gpu_util import Pair, dev, say

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("hd", [64, 128])
def test_append_decode_and_chunks_bit_exact(gpu, hd):
    say(f"append hd={hd}")
    rng = np.random.default_rng(hd)
    n_seq, n_kv = 3, 8
    p = Pair(n_seq, n_kv, hd, 300, 500000.0)
    # unaligned prefill, single-token appends, then a chunk straddling block boundaries
    for n in (45, 1, 1, 1, 37, 1, 64, 1):
        k = rng.standard_normal((n_seq, n, n_kv, hd), dtype=np.float32)
        v = rng.standard_normal((n_seq, n, n_kv, hd), dtype=np.float32)
        p.append(k, v)
        p.advance(n)
    p.check_codes()


def test_append_ragged_lengths(gpu):
    say("append ragged")
    rng = np.random.default_rng(7)
    n_seq, n_kv, hd = 5, 2, 128
    p = Pair(n_seq, n_kv, hd, 200, 1e6)
    p.set_lens([0, 31, 32, 33, 100])
    for n in (1, 40):
        k = rng.standard_normal((n_seq, n, n_kv, hd), dtype=np.float32) * 3
        v = rng.standard_normal((n_seq, n, n_kv, hd), dtype=np.float32) * 0.01
        p.append(k, v)
        p.advance(n)
    # positions below each sequence's starting length were never written on either side
    p.check_codes()


def test_append_special_values_bit_exact(gpu):
    say("append special values")
    n_kv, hd = 4, 128
    p = Pair(1, n_kv, hd, 64, 10000.0)
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, 8, n_kv, hd), dtype=np.float32)
    v = rng.standard_normal((1, 8, n_kv, hd), dtype=np.float32)
    v[0, 0, 0] = 0.0                                   # zero vector -> scale 1, 0x88888888
    v[0, 0, 1] = 1000.0                                # all equal -> 0xFFFFFFFF
    v[0, 0, 2, :3] = [np.nan, 5.0, -np.inf]            # NaN skipped by max, inf scale
    v[0, 0, 3] = rng.standard_normal(hd).astype(np.float32) * np.float32(1e-39)  # subnormals
    v[0, 1, 0] = np.tile(np.array([7, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5], np.float32), hd // 8)  # ties
    v[0, 1, 1] = (np.arange(hd, dtype=np.float32) * np.float32(0.1) - np.float32(3.15))  # reference ramp
    k[0, 2, :, :] = 0.0
    k[0, 3, 0, :] = np.float32(3.4e38)                 # near f32 max
    p.append(k, v)
    p.advance(8)
    p.check_codes()
    kp, vp, ks, vs = p.gpu.export(0, 0, 0, 1)
    vp = vp.cpu().numpy().view(np.uint32)
    assert (vp[0, 0] == 0x88888888).all() and vs[0, 0].item() == 1.0
    assert (vp[0, 1] == 0xFFFFFFFF).all()


def test_append_quotients_at_rounding_boundaries(gpu):
    """Quotients x/scale within a few ulps of the half-integers (where round() flips) under
    scales that are not powers of two, and scales at the ends of f32's range: the device's
    reciprocal shortcut must fall back to the correctly rounded division there."""
    say("append rounding boundaries")
    n_kv, hd, n_tok = 4, 128, 64
    rng = np.random.default_rng(11)
    v = np.empty((1, n_tok, n_kv, hd), np.float32)
    for t in range(n_tok):
        for h in range(n_kv):
            exp = [-120, -60, -3, 0, 5, 40, 100, 124][(t + h) % 8]
            m = np.float32(7.0 * (1.0 + rng.random()) * 2.0 ** exp)
            sc = np.float32(m / np.float32(7.0))
            half = (rng.integers(0, 7, hd) + 0.5) * rng.choice([-1.0, 1.0], hd)
            x = (half * sc).astype(np.float32)
            ulps = rng.integers(-3, 4, hd)
            for _ in range(3):  # step each value by -3..3 ulps
                x = np.where(ulps > 0, np.nextafter(x, np.float32(np.inf)), x)
                x = np.where(ulps < 0, np.nextafter(x, np.float32(-np.inf)), x)
                ulps = ulps - np.sign(ulps)
            x[0] = m
            v[0, t, h] = np.clip(x, -m, m)
    v[0, 0, 0] = np.float32(3.3e38) * np.sign(v[0, 0, 0])  # reciprocal would overflow
    v[0, 1, 0, 0] = np.float32(2e-38)                          # denormal scale
    v[0, 1, 0, 1:] = v[0, 1, 0, 1:] * np.float32(0.0)
    k = v.copy()
    p = Pair(1, n_kv, hd, n_tok + 8, 10000.0)
    p.append(k, v)
    p.advance(n_tok)
    p.check_codes()


def test_reference_known_answers_through_gpu(gpu):
    """test_int4_parity.rs cases, run through the GPU append at position 0 (rotation = identity)
    as V (never rotated) and K."""
    say("append KATs")
    with open(os.path.join(GOLD, "reference_kat.json")) as f:
        cases = json.load(f)["cases"]
    hd = 64
    for c in cases:
        x = np.array(c["x"], np.float32)
        x = np.tile(x, hd // x.size)[:hd] if x.size < hd else x
        p = Pair(1, 1, hd, 8, 10000.0)
        p.append(x.reshape(1, 1, 1, hd), x.reshape(1, 1, 1, hd))
        p.advance(1)
        p.check_codes()
        kp, vp, ks, vs = p.gpu.export(0, 0, 0, 1)
        for words, sc in ((kp, ks), (vp, vs)):
            w = words.cpu().numpy().view(np.uint32).ravel()
            s = np.float32(sc.cpu().item())
            if "expect_words" in c:
                assert (w == c["expect_words"][0]).all(), c["name"]
            if "expect_scale" in c:
                assert s == c["expect_scale"]
            nib = ((w[:, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF).ravel()
            deq = (nib.astype(np.float32) - 8) * s
            bound = 1.0 if "+ 1.0" in c.get("roundtrip_bound", "") else 1e-5
            assert np.abs(deq - x).max() <= s / 2 + bound


@pytest.mark.parametrize("with_rope", [False, True])
def test_requant_all_matches_oracle(gpu, with_rope):
    """requantize_all_kv_int4 (layer.rs:1161-1246) over an f32 cache."""
    say(f"requant rope={with_rope}")
    from oracle import oracle
    rng = np.random.default_rng(11)
    n_seq, n_kv, hd, L, ld = 2, 8, 128, 77, 90
    p = Pair(n_seq, n_kv, hd, 128, 500000.0)
    kc = rng.standard_normal((n_seq, ld, n_kv, hd), dtype=np.float32)
    vc = rng.standard_normal((n_seq, ld, n_kv, hd), dtype=np.float32)
    p.gpu.requantize_all_kv_int4(0, dev(kc), dev(vc), L, p.rope if with_rope else None)
    if with_rope:
        p.ora.append(kc[:, :L], vc[:, :L])
    else:
        ident = np.zeros_like(p.ora.table)
        ident[:, :, 0] = 1.0
        saved = p.ora.table
        p.ora.table = ident
        p.ora.append(kc[:, :L], vc[:, :L])
        p.ora.table = saved
    p.check_codes(upto=[L] * n_seq)
    del oracle


def test_overflow_and_bad_calls(gpu):
    say("overflow")
    p = Pair(2, 2, 64, 4, 10000.0)
    k = np.zeros((2, 3, 2, 64), np.float32)
    p.append(k, k)
    p.advance(3)
    with pytest.raises(TsError) as e:
        p.gpu.increment(2)  # kv_cache.rs:284-293 returns Err past max_seq_len
    assert e.value.code == _lib.TS_ERR_OVERFLOW
    assert p.gpu.get_seq_len(0) == 3  # failed increment changes nothing
    with pytest.raises(TsError) as e:
        p.gpu.append_quant(0, dev(k), dev(k), p.rope)  # 3 + 3 > 4
    assert e.value.code == _lib.TS_ERR_OVERFLOW
    with pytest.raises(TsError) as e:
        p.gpu.set_seq_len(5, seq=1)
    assert e.value.code == _lib.TS_ERR_OVERFLOW
    p.gpu.increment(1)
    assert p.gpu.seq_lens() == [4, 4]
    p.gpu.reset()
    assert p.gpu.seq_lens() == [0, 0]
    with pytest.raises(TsError):
        p.gpu.append_quant(1, dev(k), dev(k), p.rope)  # layer out of range
    torch.cuda.synchronize()
