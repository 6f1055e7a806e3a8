"""GPU tests of the cache bookkeeping around the hot path: requantization with a QK norm set,
per-sequence reset of a compacted slot, a shift that moves nothing, and the host-side checks of
caller-supplied outputs.  Codes and scales bit-exact against the oracle; attention outputs
within |err| <= 2e-3 + 1e-3*|ref|."""
import ctypes

import numpy as np
import pytest
import torch

from airframe_amd import TsError, _lib, synth
from airframe_amd.kv_cache import _stream
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu


def fill(p: Pair, rng, n, step=128):
    done = 0
    while done < n:
        m = min(step, n - done)
        p.append(synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd)), synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd)))
        p.advance(m)
        done += m


def fused_step(p: Pair, rng, n_head):
    k = synth.normal(rng, (p.n_seq, 1, p.n_kv, p.hd))
    v = synth.normal(rng, (p.n_seq, 1, p.n_kv, p.hd))
    q = synth.normal(rng, (p.n_seq, n_head, p.hd))
    out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope).cpu().numpy()
    p.ora.append(k, v)
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    p.advance(1)
    return out, ref


def test_requant_all_takes_k_as_given_with_qk_norm(gpu):
    """requantize_all_kv_int4 (layer.rs:1161-1246) quantizes the f32 cache it is given: the
    reference normalizes that cache before, so a layer's QK norm must not be applied again."""
    say("requant with qk norm set")
    rng = np.random.default_rng(21)
    n_seq, n_kv, hd, L, ld = 2, 4, 128, 70, 80
    p = Pair(n_seq, n_kv, hd, 128, 1000000.0)
    wq = torch.from_numpy((rng.standard_normal(hd) * 0.2 + 1.0).astype(np.float32)).cuda()
    wk = torch.from_numpy((rng.standard_normal(hd) * 0.2 + 1.0).astype(np.float32)).cuda()
    p.gpu.set_qk_norm(0, wq, wk)
    kc = rng.standard_normal((n_seq, ld, n_kv, hd), dtype=np.float32)
    vc = rng.standard_normal((n_seq, ld, n_kv, hd), dtype=np.float32)
    p.gpu.requantize_all_kv_int4(0, dev(kc), dev(vc), L, p.rope)
    p.ora.append(kc[:, :L], vc[:, :L])  # the oracle has no norm set: K as given, rotated
    p.check_codes(upto=[L] * n_seq)


@pytest.mark.parametrize("hd", [64, 128])
def test_reset_one_compacted_sequence(gpu, hd):
    """KVCache::reset (kv_cache.rs:256-259) zeroes window_base with the length: a reused,
    compacted slot must start like a fresh cache while the other sequences keep theirs."""
    say(f"reset_seq hd={hd}")
    rng = np.random.default_rng(40 + hd)
    n_head = 8
    p = Pair(3, 2, hd, 400, 10000.0, rope_n_pos=1200)
    fill(p, rng, 200)
    # compact sequence 1 (window base 90, 4 sinks), as the reference's caller does
    p.gpu.compact(4, 90, seq=1)
    p.ora.shift(1, 4, 90)
    p.ora.advance_window_base(1, 90)
    p.ora.lens[1] -= 90
    assert p.gpu.get_window_base(1) == 90
    # reuse slot 1 for a new sequence
    p.gpu.reset(seq=1)
    p.ora.lens[1] = 0
    p.ora.rot[1] = 0
    p.ora.n_sink[1] = 0
    assert p.gpu.get_window_base(1) == 0 and p.gpu.get_seq_len(1) == 0
    assert p.gpu.get_window_base(0) == 0 and p.gpu.get_seq_len(0) == 200
    fill(p, rng, 70)  # appends at 200 / 0 / 200
    p.check_codes()
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head)
        assert_close(out, ref, "fused decode after a per-sequence reset")
    p.check_codes()
    # a new first shift on the reset slot may pick another sink count
    p.gpu.shift_int4(0, 2, 10, seq=1)
    p.ora.shift(1, 2, 10)
    p.check_codes(upto=[p.ora.lens[0], p.ora.lens[1] - 10, p.ora.lens[2]])


def test_shift_that_moves_nothing_records_sinks(gpu):
    """A first shift with len <= keep_sink + shift_amt moves nothing but records the sink
    count, so advancing the window base after it (the reference caller's order) keeps the
    sinks at their own rotation and later shifts with the same keep_sink are accepted."""
    say("shift moving nothing")
    rng = np.random.default_rng(77)
    n_head = 8
    p = Pair(2, 2, 128, 300, 10000.0, rope_n_pos=900)
    fill(p, rng, 30)
    p.gpu.shift_int4(0, 4, 40, seq=0)   # 30 <= 4 + 40: nothing moves
    p.ora.shift(0, 4, 40)
    p.gpu.advance_window_base(40, seq=0)
    p.ora.advance_window_base(0, 40)
    p.check_codes()
    fill(p, rng, 20)  # sequence 0 appends rotated at slot + 40, its 4 sinks stay put
    p.check_codes()
    out, ref = fused_step(p, rng, n_head)
    assert_close(out, ref, "fused decode after a shift that moved nothing")
    with pytest.raises(TsError):
        p.gpu.shift_int4(0, 2, 5, seq=0)  # another sink count
    p.gpu.shift_int4(0, 4, 5, seq=0)
    p.ora.shift(0, 4, 5)
    p.check_codes(upto=[p.ora.lens[0] - 5, p.ora.lens[1]])


def _shift_raw(p: Pair, seq, keep_sink, shift_amt, ws=None, ws_bytes=0):
    return _lib.load().ts_kv_shift(p.gpu.handle, 0, seq, keep_sink, shift_amt, ws, ws_bytes, _stream())


def test_refused_shift_changes_nothing(gpu):
    """A shift that needs the workspace (more than 8 in-place rounds) and gets none is refused
    before the sink count is recorded: a later first shift with another sink count is still
    accepted.  A shift of at most 8 rounds runs in place with no workspace at all."""
    say("shift refused without workspace")
    rng = np.random.default_rng(78)
    p = Pair(2, 2, 128, 300, 10000.0, rope_n_pos=900)
    fill(p, rng, 200)
    # seq 0: keep 4, shift 10 -> 186 moved slots in 19 rounds: needs the workspace
    assert _shift_raw(p, 0, 4, 10) == _lib.TS_ERR_WORKSPACE
    p.check_codes()  # nothing moved
    # seq 0 takes another sink count (none was recorded), in place without a workspace:
    # keep 2, shift 100 -> 98 moved slots in one round
    assert _shift_raw(p, 0, 2, 100) == _lib.TS_OK
    p.ora.shift(0, 2, 100)
    p.check_codes(upto=[p.ora.lens[0] - 100, p.ora.lens[1]])


def test_output_shapes_are_checked(gpu):
    """Caller-supplied outputs of the wrong size raise before anything is launched."""
    say("output shape checks")
    rng = np.random.default_rng(5)
    p = Pair(2, 2, 64, 64, 10000.0)
    fill(p, rng, 8)
    q = dev(synth.normal(rng, (2, 8, 64)))
    k = dev(synth.normal(rng, (2, 1, 2, 64)))
    small = torch.empty((2, 8, 32), device="cuda")
    with pytest.raises(ValueError):
        p.gpu.attn_decode(0, q, p.rope, out=small)
    with pytest.raises(ValueError):
        p.gpu.attn_decode_append(0, k, k, q, p.rope, out=small)
    with pytest.raises(ValueError):
        p.gpu.attn_prefill(0, dev(synth.normal(rng, (2, 3, 8, 64))), p.rope,
                           out=torch.empty((2, 3, 8, 63), device="cuda"))
    assert p.gpu.seq_lens() == [8, 8]


def test_reference_buffer_getters(gpu):
    """get_{k,v}_{packed,scale}_buffer (kv_cache.rs:312-345) as copies of one sequence's whole
    layer in the reference layout, and calculate_offset (:366-369)."""
    say("buffer getters")
    rng = np.random.default_rng(8)
    p = Pair(2, 2, 64, 96, 10000.0)
    fill(p, rng, 40)
    full = [t.cpu() for t in p.gpu.export(0, 1, 0, 96)]
    got = [p.gpu.get_k_packed_buffer(0, seq=1), p.gpu.get_v_packed_buffer(0, seq=1),
           p.gpu.get_k_scale_buffer(0, seq=1), p.gpu.get_v_scale_buffer(0, seq=1)]
    for a, b in zip(full, got):
        assert tuple(b.shape) == tuple(a.shape) and torch.equal(a.view(torch.uint8), b.cpu().view(torch.uint8))
    assert tuple(got[0].shape) == (96, 2, 8) and tuple(got[2].shape) == (96, 2)
    p.check_codes()
    assert p.gpu.calculate_offset(0, 0, 0) == 0
    assert p.gpu.calculate_offset(3, 1, 5) == ((3 * 2 + 1) * 64 + 5) * 4
