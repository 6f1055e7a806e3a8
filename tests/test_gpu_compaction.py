"""GPU parity of sliding-window compaction (RopeShiftPipeline::execute_int4, KVCache window
base): after ts_kv_shift the cache holds the oracle's codes and scales bit-exact (a pure copy of
the moved slots), and decode, fused decode and prefill after one or two compactions match the
oracle, whose compaction semantics are pinned against the reference's relative-RoPE attention
with sinks in tests/test_oracle.py.  |err| <= 2e-3 + 1e-3*|ref| for outputs."""
import numpy as np
import pytest

from airframe_amd import TsError, synth
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu


def compact(p: Pair, seq: int, keep: int, amt: int):
    n = int(p.ora.lens[seq])
    p.gpu.compact(keep, amt, seq)
    if n > keep + amt and amt > 0:
        p.ora.shift(seq, keep, amt)
        p.ora.advance_window_base(seq, amt)
        p.ora.lens[seq] = n - amt


def fill(p: Pair, rng, n, step=256):
    done = 0
    while done < n:
        m = min(step, n - done)
        k = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd))
        v = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd))
        p.append(k, v)
        p.advance(m)
        done += m


def fused_step(p: Pair, rng, n_head, softcap=0.0):
    k = synth.normal(rng, (p.n_seq, 1, p.n_kv, p.hd))
    v = synth.normal(rng, (p.n_seq, 1, p.n_kv, p.hd))
    q = synth.normal(rng, (p.n_seq, n_head, p.hd))
    out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope, softcap=softcap).cpu().numpy()
    p.ora.append(k, v)
    ref = p.ora.attend(q[:, None], 1, softcap=softcap, threads=8)[:, 0]
    p.advance(1)
    return out, ref


def prefill_chunk(p: Pair, rng, n_head, n_tok):
    k = synth.normal(rng, (p.n_seq, n_tok, p.n_kv, p.hd))
    v = synth.normal(rng, (p.n_seq, n_tok, p.n_kv, p.hd))
    q = synth.normal(rng, (p.n_seq, n_tok, n_head, p.hd))
    p.append(k, v)
    out = p.gpu.attn_prefill(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q, n_tok, threads=8)
    p.advance(n_tok)
    return out, ref


@pytest.mark.parametrize("hd", [64, 128])
def test_shift_then_decode_and_prefill(gpu, hd):
    say(f"compaction hd={hd}")
    rng = np.random.default_rng(300 + hd)
    n_head = 8
    p = Pair(3, 2, hd, 320, 10000.0, rope_n_pos=1400)
    fill(p, rng, 250)
    p.set_lens([250, 200, 150])
    compact(p, 0, 4, 100)   # moved block boundaries do not line up with 32-position V blocks
    compact(p, 1, 4, 37)
    compact(p, 2, 4, 146)   # 150 <= 4 + 146: nothing moves
    assert [p.gpu.get_window_base(s) for s in range(3)] == [100, 37, 0]
    p.check_codes()
    for _ in range(3):
        out, ref = fused_step(p, rng, n_head)
        assert_close(out, ref, "fused decode after compaction")
    out, ref = prefill_chunk(p, rng, n_head, 21)
    assert_close(out, ref, "prefill after compaction")
    compact(p, 0, 4, 60)    # a second compaction: window base 160
    compact(p, 1, 4, 1)
    p.check_codes()
    out, ref = fused_step(p, rng, n_head, softcap=20.0)
    assert_close(out, ref, "fused decode after second compaction")
    p.check_codes()


def test_separate_append_and_decode_after_compaction(gpu):
    say("compaction separate calls")
    rng = np.random.default_rng(310)
    n_head = 12
    p = Pair(2, 4, 128, 700, 500000.0, rope_n_pos=2000)
    fill(p, rng, 600)
    compact(p, 0, 4, 333)
    compact(p, 1, 4, 64)
    k = synth.normal(rng, (2, 1, 4, 128))
    v = synth.normal(rng, (2, 1, 4, 128))
    q = synth.normal(rng, (2, n_head, 128))
    p.append(k, v)
    out = p.gpu.attn_decode(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    assert_close(out, ref, "decode after compaction")
    p.advance(1)
    p.check_codes()


@pytest.mark.parametrize("n_head", [32, 64, 128])
def test_long_split_kernel_after_compaction(gpu, n_head):
    """32 sequences x 8 kv heads at ~4200 slots after compaction: the integer-QK decode kernel
    (one split per stream) with 4, 8 and 16 query heads per kv head."""
    say(f"compaction long splits, {n_head} q heads")
    rng = np.random.default_rng(320 + n_head)
    p = Pair(32, 8, 128, 5200, 1e6, rope_n_pos=6200)
    fill(p, rng, 5000, step=1024)
    for s in range(32):
        compact(p, s, 4, 700 + 3 * s)
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head)
        assert_close(out, ref, "long-split fused decode after compaction")
    p.check_codes()


def test_compaction_errors(gpu):
    say("compaction errors")
    rng = np.random.default_rng(330)
    p = Pair(1, 2, 64, 200, 10000.0, rope_n_pos=400)
    fill(p, rng, 150)
    compact(p, 0, 4, 50)
    with pytest.raises(TsError):
        p.gpu.shift_int4(0, 8, 10)          # a different sink count than the first shift
    tiny = dev(np.zeros(4, np.float32))
    with pytest.raises(TsError):
        p.gpu.shift_int4(0, 4, 10, workspace=tiny)
    with pytest.raises(TsError):
        p.gpu.advance_window_base(-1)
    p.gpu.shift_int4(0, 4, 0)               # shift of 0: nothing to do
    p.check_codes()
    p.gpu.reset()
    assert p.gpu.get_window_base(0) == 0
