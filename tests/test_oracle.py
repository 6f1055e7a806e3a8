"""Pins the CPU oracle (oracle/ts_oracle.c) before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle fails it: the reference's own
known answers (test_int4_parity.rs), closed forms of RoPE and attention, and an independent
numpy restatement (oracle/np_oracle.py) on small inputs.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import np_oracle, oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _kat():
    with open(os.path.join(GOLD, "reference_kat.json")) as f:
        return {c["name"]: c for c in json.load(f)["cases"]}


# ---- quantizer: reference known answers (test_int4_parity.rs) ---------------------------------

def test_kat_zero_vector():  # :489-520
    c = _kat()["zero_vector_no_nan"]
    s, w = oracle.quantize_row(np.array(c["x"], np.float32))
    assert s == np.float32(1.0) and np.isfinite(s)
    assert list(w) == c["expect_words"] == [0x88888888]


def test_kat_extreme_all_positive():  # :525-572
    c = _kat()["extreme_all_positive"]
    s, w = oracle.quantize_row(np.array(c["x"], np.float32))
    assert list(w) == [0xFFFFFFFF]
    assert s == np.float32(1000.0) / np.float32(7.0)


@pytest.mark.parametrize("name,bound_abs", [
    ("extreme_alternating", 1.0), ("single_head_ramp_k", 1e-5), ("single_head_sinusoid_v", 1e-5)]
    + [(f"multi_head_k_amp{a}", 1e-5) for a in (1.0, 2.0, 0.5, 7.0)]
    + [(f"multi_head_v_amp{a}", 1e-5) for a in (1.0, 2.0, 0.5, 7.0)])
def test_kat_roundtrip_bound(name, bound_abs):  # :370-385, :455-473, :575-581
    c = _kat()[name]
    x = np.array(c["x"], np.float32)
    s, w = oracle.quantize_row(x)
    err = np.abs(oracle.dequantize_row(w, s) - x).max()
    assert err <= s / 2 + bound_abs
    if "expect_scale_close" in c:  # multi-head: independent per-head scales amp*max|..|/7
        assert abs(s - c["expect_scale_close"]) < 1e-5
    if "expect_max_abs" in c:  # ramp: max_abs 3.15 -> scale ~0.45
        assert abs(s * 7 - c["expect_max_abs"]) < 1e-5


def test_kat_ramp_words_by_hand():
    # ramp d*0.1-3.15, scale = 3.15/7 = 0.45: element 0 is -3.15/0.45 = -7 -> code 1;
    # element 31 is -0.05/0.45 -> round(-0.111) = 0 -> code 8; element 63 -> +7 -> 15.
    x = np.array(_kat()["single_head_ramp_k"]["x"], np.float32)
    s, w = oracle.quantize_row(x)
    nib = lambda i: (int(w[i // 8]) >> (4 * (i % 8))) & 0xF  # noqa: E731
    assert nib(0) == 1 and nib(31) == 8 and nib(63) == 15
    # d=4: -2.75/0.45 = -6.11 -> -6 -> 2 ;  d=5: -2.65/0.45=-5.89 -> -6 -> 2
    assert nib(4) == 2 and nib(5) == 2


def test_quantizer_layout_and_rounding_by_hand():
    # scale = 7/7 = 1: codes are round_half_away(x) + 8, element n of a word at bits 4n.
    x = np.array([7, -7, 0.5, -0.5, 1.5, -1.5, 2.49, 0], np.float32)
    s, w = oracle.quantize_row(x)
    assert s == 1.0
    # half away from zero: 0.5 -> 1, -0.5 -> -1, 1.5 -> 2, -1.5 -> -2
    codes = [15, 1, 9, 7, 10, 6, 10, 8]
    assert int(w[0]) == sum(c << (4 * n) for n, c in enumerate(codes))


def test_quantizer_special_values():
    # NaN is skipped by the max (f32::max) and encodes as code 8 (NaN as i32 == 0);
    # +inf makes scale inf: finite/inf = 0 -> 8, inf/inf = NaN -> 8.
    x = np.array([np.nan, 2.0, -3.5, 0, 0, 0, 0, 1.0], np.float32)
    s, w = oracle.quantize_row(x)
    assert s == np.float32(3.5) / np.float32(7.0)
    assert int(w[0]) & 0xF == 8
    x = np.array([np.inf, 1.0, -1.0, 0, 0, 0, 0, 0], np.float32)
    s, w = oracle.quantize_row(x)
    assert np.isinf(s) and int(w[0]) == 0x88888888
    # subnormal max: scale stays subnormal, codes still span [1,15]
    x = np.array([1e-40, -1e-40, 5e-41, 0, 0, 0, 0, 0], np.float32)
    s, w = oracle.quantize_row(x)
    assert 0 < s < np.finfo(np.float32).tiny
    assert (int(w[0]) & 0xF) == 15 and ((int(w[0]) >> 4) & 0xF) == 1


def test_quantizer_invariants_random():
    rng = np.random.default_rng(5)
    for hd in (8, 64, 128):
        x = (rng.standard_normal((200, hd)) * rng.uniform(0.01, 100, (200, 1))).astype(np.float32)
        for row in x:
            s, w = oracle.quantize_row(row)
            nib = (w[:, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF
            assert nib.min() >= 1 and nib.max() <= 15
            assert np.abs(oracle.dequantize_row(w, s) - row).max() <= s / 2 * (1 + 1e-6)


def test_quantizer_matches_numpy_restatement():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((500, 128)).astype(np.float32)
    x[::7] *= 1000
    x[3, 5] = 0.5 * 7 / 7  # ties appear naturally too; both use half-away rounding
    ref_s, ref_w = np_oracle.quantize(x)
    for i, row in enumerate(x):
        s, w = oracle.quantize_row(row)
        assert s == ref_s[i] and (w == ref_w[i]).all()


def test_tie_rounding_half_away():
    # x/scale == +-2.5 exactly: half away gives +-3 (codes 11 and 5); half-even would give +-2.
    x = np.array([7.0, 2.5, -2.5, 0, 0, 0, 0, 0], np.float32)
    s, w = oracle.quantize_row(x)
    assert ((int(w[0]) >> 4) & 0xF) == 11 and ((int(w[0]) >> 8) & 0xF) == 5
    s2, w2 = np_oracle.quantize(x)
    assert (w2 == w).all()


# ---- RoPE ---------------------------------------------------------------------------------------

def test_rope_table_closed_forms():
    t = oracle.rope_table(64, 128, 500000.0)
    assert (t[0, :, 0] == 1.0).all() and (t[0, :, 1] == 0.0).all()  # preflight.rs:267-285
    # pair 0 has theta 1: angle = pos
    assert np.allclose(t[:, 0, 0], np.cos(np.arange(64)), atol=1e-6)
    # theta_i = base^(-2i/d) in float64 within f32 rounding (closed form)
    i = np.arange(64)
    theta = 500000.0 ** (-2.0 * i / 128)
    assert np.allclose(t[5, :, 0], np.cos(5 * theta), atol=2e-6)
    assert np.allclose(t[5, :, 1], np.sin(5 * theta), atol=2e-6)
    # linear scale multiplies theta (preflight.rs:288-303)
    t2 = oracle.rope_table(8, 8, 10000.0, 2.0)
    assert np.allclose(t2[3, 0], [np.cos(6.0), np.sin(6.0)], atol=1e-6)
    with pytest.raises(ValueError):
        oracle.rope_table(8, 8, 10000.0, 0.0)


def test_rope_table_reference_vectors():
    """The reference's own table tests (preflight.rs:266-331)."""
    # distance 0 is (1, 0) whatever the scaling (:266-285)
    for args in [(4, 4, 10000.0, 1.0), (4, 4, 10000.0, 0.5), (4000, 4, 1.0001, 0.5, 0.1, 1.0)]:
        t = oracle.rope_table(*args)
        assert (np.abs(t[0, :, 0] - 1.0) < 1e-6).all() and (np.abs(t[0, :, 1]) < 1e-6).all()
    # linear scale 0.5, no YaRN parameters: pair 0 at distance 1 is cos(0.5) (:287-302)
    t = oracle.rope_table(4, 4, 10000.0, 0.5)
    assert abs(t[1, 0, 0] - np.cos(np.float32(0.5))) < 1e-6
    # YaRN with a tiny base: pair 0 is a short wavelength, its ramp clamps to 1 and it keeps
    # theta unscaled, cos(1), unlike the linear table's cos(0.5) (:304-331)
    ty = oracle.rope_table(4000, 4, 1.0001, 0.5, 0.1, 1.0)
    tl = oracle.rope_table(4000, 4, 1.0001, 0.5)
    assert abs(ty[1, 0, 0] - tl[1, 0, 0]) > 1e-3
    assert abs(ty[1, 0, 0] - np.cos(1.0)) < 1e-4


def test_rope_table_yarn_ramp_ends_and_transition():
    """YaRN's two ends reduce to the plain tables: pairs whose ramp clamps to 1 equal the
    unscaled table bit for bit (factor (1-1) s + 1 = 1), pairs clamped to 0 equal the linear one
    (factor s).  Between them the factor falls monotonically, and where each end starts pins
    l_train = round(n_pos * scale) and the roles of alpha and beta."""
    n_pos, d, base, s, a, b = 8192, 128, 500000.0, 0.25, 1.0, 32.0
    ty = oracle.rope_table(n_pos, d, base, s, a, b)
    t1 = oracle.rope_table(n_pos, d, base, 1.0)
    ts = oracle.rope_table(n_pos, d, base, s)
    i = np.arange(d // 2)
    theta = base ** (-2.0 * i / d)
    x = round(n_pos * s) * theta / (2 * np.pi)  # l_train / wavelength, float64
    hi, lo = x >= b * 1.001, x <= a * 0.999
    assert hi.sum() >= 3 and lo.sum() >= 3 and (~hi & ~lo).sum() >= 3
    assert np.array_equal(ty[:, hi].view(np.uint32), t1[:, hi].view(np.uint32))
    assert np.array_equal(ty[:, lo].view(np.uint32), ts[:, lo].view(np.uint32))
    # effective theta from the table: angle at distance 1
    eff = np.arctan2(ty[1, :, 1], ty[1, :, 0]).astype(np.float64) / theta
    mid = ~hi & ~lo
    assert ((eff[mid] > s) & (eff[mid] < 1.0)).all()
    assert (np.diff(eff[mid]) < 0).all()  # ramp falls as the wavelength grows
    # a linear ramp in x between the ends: factor = s + (1 - s) (x - a) / (b - a)
    assert np.allclose(eff[mid], s + (1 - s) * (x[mid] - a) / (b - a), rtol=2e-5)


def test_rope_rotation_is_pairwise_rotation():
    rng = np.random.default_rng(2)
    t = oracle.rope_table(100, 64, 10000.0)
    x = rng.standard_normal(64).astype(np.float32)
    y = oracle.rope_rotate(x, t[37])
    # norm per pair preserved, angle advanced by 37*theta_i
    for i in range(32):
        a, b = x[2 * i], x[2 * i + 1]
        c, s = t[37, i]
        assert abs(y[2 * i] - (a * c - b * s)) < 1e-6 and abs(y[2 * i + 1] - (a * s + b * c)) < 1e-6
        assert abs(math.hypot(y[2 * i], y[2 * i + 1]) - math.hypot(a, b)) < 1e-5
    # adjacent pairs (2i, 2i+1), not halves: rotating e0 only moves dims 0 and 1
    e0 = np.zeros(64, np.float32)
    e0[0] = 1
    y = oracle.rope_rotate(e0, t[3])
    assert np.count_nonzero(y) <= 2 and y[1] != 0
    # relative-position identity used by the reference GPU kernel (sh_layer_v1_int4.wgsl:1112)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    d1 = np.dot(oracle.rope_rotate(q, t[50]), oracle.rope_rotate(k, t[20]))
    d2 = np.dot(oracle.rope_rotate(q, t[31]), oracle.rope_rotate(k, t[1]))
    assert abs(d1 - d2) < 1e-4


# ---- attention ------------------------------------------------------------------------------------

def _cache(n_seq, max_seq, n_kv, hd, base=10000.0):
    return oracle.OracleKV(n_seq, max_seq, n_kv, hd, oracle.rope_table(max_seq, hd, base))


def test_attention_single_position_is_v():
    kv = _cache(1, 4, 2, 64)
    rng = np.random.default_rng(0)
    k = rng.standard_normal((1, 1, 2, 64), dtype=np.float32)
    v = rng.standard_normal((1, 1, 2, 64), dtype=np.float32)
    kv.append(k, v)
    q = rng.standard_normal((1, 1, 4, 64), dtype=np.float32)
    out = kv.attend(q, 1)
    for h in range(4):
        vd = oracle.dequantize_row(kv.v_packed[0, 0, h // 2], kv.v_scale[0, 0, h // 2])
        assert (out[0, 0, h] == vd).all()  # p == 1 exactly, f64 sum of 1*v


def test_attention_equal_keys_give_mean_and_gqa_mapping():
    n_kv, G, hd, L = 2, 3, 64, 10
    kv = _cache(1, L, n_kv, hd)
    rng = np.random.default_rng(1)
    k = np.zeros((1, L, n_kv, hd), np.float32)  # all keys zero -> all scores equal
    v = rng.standard_normal((1, L, n_kv, hd), dtype=np.float32)
    v[0, :, 1] += 100.0  # kv head 1 clearly distinct from head 0
    kv.append(k, v)
    kv.advance(L - 1)
    kv.lens[:] = L - 1
    q = rng.standard_normal((1, 1, n_kv * G, hd), dtype=np.float32)
    out = kv.attend(q, 1)
    for h in range(n_kv * G):
        kvh = h // G  # attention.rs:237
        vd = np.stack([oracle.dequantize_row(kv.v_packed[0, j, kvh], kv.v_scale[0, j, kvh]) for j in range(L)])
        assert np.allclose(out[0, 0, h], vd.mean(0), atol=1e-5)


def test_attention_two_keys_closed_form():
    # scores s0, s1 -> weights sigmoid(s0-s1); check the 1/sqrt(hd) factor and the softmax.
    hd = 64
    kv = _cache(1, 2, 1, hd, base=1e30)  # base so large every angle is ~0 beyond pair 0
    t = kv.table
    t[:] = 0
    t[:, :, 0] = 1.0  # identity rotation
    k = np.zeros((1, 2, 1, hd), np.float32)
    k[0, 0, 0, 0] = 7.0
    k[0, 1, 0, 0] = -7.0
    v = np.zeros((1, 2, 1, hd), np.float32)
    v[0, 0, 0, :] = 7.0
    v[0, 1, 0, :] = -7.0
    kv.append(k, v)
    kv.lens[:] = 1
    q = np.zeros((1, 1, 1, hd), np.float32)
    q[0, 0, 0, 0] = 2.0
    out = kv.attend(q, 1)
    s0, s1 = 2 * 7 / math.sqrt(hd), -2 * 7 / math.sqrt(hd)
    w0 = 1 / (1 + math.exp(s1 - s0))
    assert abs(out[0, 0, 0, 3] - (7 * w0 - 7 * (1 - w0))) < 1e-5


def test_attention_decode_equals_last_prefill_row():  # kvcache.rs:363-416
    rng = np.random.default_rng(3)
    n_kv, n_head, hd, L = 2, 4, 64, 33
    a = _cache(1, L, n_kv, hd)
    b = _cache(1, L, n_kv, hd)
    k = rng.standard_normal((1, L, n_kv, hd), dtype=np.float32)
    v = rng.standard_normal((1, L, n_kv, hd), dtype=np.float32)
    q = rng.standard_normal((1, L, n_head, hd), dtype=np.float32)
    a.append(k, v)
    full = a.attend(q, L)
    b.append(k[:, :-1], v[:, :-1])
    b.advance(L - 1)
    b.append(k[:, -1:], v[:, -1:])
    last = b.attend(q[:, -1:], 1)
    assert np.array_equal(full[:, -1:], last)
    # causal: the first query only sees key 0 -> output is V[0]
    vd0 = oracle.dequantize_row(a.v_packed[0, 0, 0], a.v_scale[0, 0, 0])
    assert (full[0, 0, 0] == vd0).all()


def test_attention_matches_numpy_restatement():
    rng = np.random.default_rng(4)
    n_kv, n_head, hd, L, T = 2, 6, 128, 50, 7
    kv = _cache(2, L + T, n_kv, hd, base=1e6)
    k = rng.standard_normal((2, L + T, n_kv, hd), dtype=np.float32)
    v = rng.standard_normal((2, L + T, n_kv, hd), dtype=np.float32)
    kv.append(k[:, :L], v[:, :L])
    kv.advance(L)
    kv.append(k[:, L:], v[:, L:])
    q = rng.standard_normal((2, T, n_head, hd), dtype=np.float32)
    for softcap in (0.0, 5.0):
        out = kv.attend(q, T, softcap=softcap)
        out_mt = kv.attend(q, T, softcap=softcap, threads=4)
        assert np.array_equal(out, out_mt)
        t = kv.table
        for s in range(2):
            kd = np_oracle.dequantize(kv.k_packed[s, :L + T], kv.k_scale[s, :L + T])
            vd = np_oracle.dequantize(kv.v_packed[s, :L + T], kv.v_scale[s, :L + T])
            qr = np_oracle.rotate(q[s], t[L:L + T, None, :, 0], t[L:L + T, None, :, 1])
            ref = np_oracle.attend(qr, kd, vd, L, softcap)
            assert np.abs(ref - out[s]).max() < 2e-6


def test_append_matches_numpy_restatement_and_keeps_v_unrotated():
    rng = np.random.default_rng(8)
    kv = _cache(1, 20, 3, 128, base=500000.0)
    k = rng.standard_normal((1, 20, 3, 128), dtype=np.float32)
    v = rng.standard_normal((1, 20, 3, 128), dtype=np.float32)
    kv.append(k, v)
    t = kv.table
    kr = np_oracle.rotate(k[0], t[:20, None, :, 0], t[:20, None, :, 1])
    ks, kw = np_oracle.quantize(kr)
    vs, vw = np_oracle.quantize(v[0])
    assert (kw == kv.k_packed[0]).all() and (ks == kv.k_scale[0]).all()
    assert (vw == kv.v_packed[0]).all() and (vs == kv.v_scale[0]).all()
    # position 0 rotation is the identity
    s0, w0 = oracle.quantize_row(k[0, 0, 1])
    assert (w0 == kv.k_packed[0, 0, 1]).all()


# ---- golden fixture -------------------------------------------------------------------------------

def test_oracle_reproduces_golden_fixture():
    g = np.load(os.path.join(GOLD, "oracle_small.npz"))
    c = json.loads(str(g["config"]))
    P, C = c["prefill"], c["chunk"]
    kv = _cache(c["n_seq"], P + C + 1, c["n_kv"], c["hd"], c["base"])
    kv.append(g["k0"], g["v0"])
    kv.advance(P)
    kv.append(g["k1"], g["v1"])
    assert np.array_equal(kv.attend(g["q1"], C), g["o_prefill"])
    kv.advance(C)
    kv.append(g["k2"], g["v2"])
    assert np.array_equal(kv.attend(g["q2"], 1), g["o_decode"])
    for name in ("k_packed", "v_packed", "k_scale", "v_scale"):
        assert np.array_equal(getattr(kv, name), g[name])


# ---- sliding-window compaction (pipeline_shift.rs, kv_cache.rs window_base) ----------------------

def _reference_relative_attention(q, k_raw, v, compact_q, window_base, n_sink, table, sink_count=4):
    """sh_layer_v1_int4.wgsl:1062-1143 restated in float64 for one head: the reference keeps
    K unrotated and applies RoPE(rel) in the score, with rel the compacted distance, except for
    the sink slots (pos < SINK_COUNT), which use the logical distance window_base + qpos - pos."""
    hd = q.shape[0]
    L = k_raw.shape[0]
    logical_q = window_base + compact_q
    scores = np.empty(L)
    for pos in range(L):
        rel = (logical_q - pos) if pos < sink_count else (compact_q - pos)
        c = table[rel, :, 0].astype(np.float64)
        s = table[rel, :, 1].astype(np.float64)
        qr, qi = q[0::2].astype(np.float64), q[1::2].astype(np.float64)
        kr, ki = k_raw[pos, 0::2], k_raw[pos, 1::2]
        scores[pos] = np.sum((qr * kr + qi * ki) * c + (qr * ki - qi * kr) * s) / math.sqrt(hd)
    p = np.exp(scores - scores.max())
    return (p / p.sum()) @ v


def test_compaction_matches_reference_relative_rope():
    """Two compactions and appends around them.  The oracle stores K rotated at its slot
    position plus the window base (sinks at their own position) and rotates q at its slot
    plus the window base; its outputs must equal the reference's relative-RoPE attention over
    the compacted slots (compacted distances for window slots, logical distances for the
    four sinks), with each slot's raw K recovered by rotating its dequantized K back."""
    rng = np.random.default_rng(21)
    n_kv, hd, n_head, max_seq = 2, 64, 4, 256
    table = oracle.rope_table(1024, hd, 10000.0)
    kv = oracle.OracleKV(1, max_seq, n_kv, hd, table)
    angle = np.zeros((1, max_seq), np.int64)  # rotation position of every slot's stored K

    def append(n):
        k = rng.standard_normal((1, n, n_kv, hd), dtype=np.float32)
        v = rng.standard_normal((1, n, n_kv, hd), dtype=np.float32)
        kv.append(k, v)
        for t in range(n):
            pos = kv.lens[0] + t
            angle[0, pos] = pos if pos < kv.n_sink[0] else pos + kv.rot[0]
        kv.advance(n)

    def shift(keep, amt):
        old = int(kv.lens[0])
        kv.shift(0, keep, amt)
        angle[0, keep:old - amt] = angle[0, keep + amt:old].copy()
        kv.advance_window_base(0, amt)
        kv.lens[0] = old - amt

    def check():
        L = int(kv.lens[0])
        q = rng.standard_normal((1, 1, n_head, hd), dtype=np.float32)
        kv.lens[0] = L - 1  # the query is the last slot: attend over 0..L-1
        out = kv.attend(q, 1)[0, 0]
        kv.lens[0] = L
        for head in range(n_head):
            h = head // (n_head // n_kv)
            k_raw = np.empty((L, hd))
            vd = np.empty((L, hd))
            for j in range(L):
                kd = oracle.dequantize_row(kv.k_packed[0, j, h], kv.k_scale[0, j, h]).astype(np.float64)
                c = table[angle[0, j], :, 0].astype(np.float64)
                s = table[angle[0, j], :, 1].astype(np.float64)
                a, b = kd[0::2], kd[1::2]
                k_raw[j, 0::2] = a * c + b * s     # inverse rotation
                k_raw[j, 1::2] = -a * s + b * c
                vd[j] = oracle.dequantize_row(kv.v_packed[0, j, h], kv.v_scale[0, j, h])
            ref = _reference_relative_attention(q[0, 0, head], k_raw, vd, L - 1, int(kv.rot[0]),
                                                int(kv.n_sink[0]), table)
            np.testing.assert_allclose(out[head], ref, rtol=1e-4, atol=1e-5)

    append(150)
    check()
    shift(4, 60)
    append(1)
    check()
    append(40)
    shift(4, 37)
    append(1)
    check()
    assert kv.rot[0] == 97 and kv.n_sink[0] == 4


def test_shift_is_a_copy():
    """sh_rope_shift_int4.wgsl:44-84: slots keep_sink+shift.. move down unchanged, sinks and
    nothing else change; a shift past the length moves nothing."""
    rng = np.random.default_rng(22)
    kv = oracle.OracleKV(2, 64, 2, 64, oracle.rope_table(128, 64, 10000.0))
    k = rng.standard_normal((2, 50, 2, 64), dtype=np.float32)
    kv.append(k, k * 2)
    kv.advance(50)
    before = [a.copy() for a in (kv.k_packed, kv.v_packed, kv.k_scale, kv.v_scale)]
    kv.shift(0, 4, 10)
    for a, b in zip((kv.k_packed, kv.v_packed, kv.k_scale, kv.v_scale), before):
        assert (a[0, :4] == b[0, :4]).all()
        assert (a[0, 4:40] == b[0, 14:50]).all()
        assert (a[0, 40:50] == b[0, 40:50]).all()  # stale tail, beyond the new length
        assert (a[1] == b[1]).all()                # other sequence untouched
    snap = [a.copy() for a in (kv.k_packed, kv.v_packed)]
    kv.shift(1, 30, 30)  # 50 <= 60: nothing moves
    assert all((a == b).all() for a, b in zip((kv.k_packed, kv.v_packed), snap))


# ---- QK norm (Qwen3, attention.rs:92-108 and :186-189) --------------------------------------------

def _qk_norm_py(x, w, eps):
    """attention.rs:92-108 with every operation rounded to float32, in the reference's order."""
    f = np.float32
    s = f(0.0)
    for v in x:
        s = f(s + f(v * v))
    scale = f(f(1.0) / f(np.sqrt(f(f(s / f(len(x))) + f(eps)))))
    return np.array([f(f(v * scale) * wd) for v, wd in zip(x, w)], np.float32)


@pytest.mark.parametrize("mag", [1e-3, 1.0, 37.0, 3e4])
def test_qk_norm_row_matches_reference_order(mag):
    rng = np.random.default_rng(int(mag * 10) + 5)
    for hd in (64, 128):
        x = (rng.standard_normal(hd) * mag).astype(np.float32)
        w = (rng.standard_normal(hd) * 0.5 + 1.0).astype(np.float32)
        got = oracle.qk_norm_row(x, w, 1e-6)
        assert np.array_equal(got.view(np.uint32), _qk_norm_py(x, w, 1e-6).view(np.uint32))


def test_qk_norm_closed_form():
    hd = 128
    w = np.linspace(0.5, 2.0, hd).astype(np.float32)
    for c in (0.0, 1.0, -3.0):
        got = oracle.qk_norm_row(np.full(hd, c, np.float32), w, 1e-6)
        want = c / math.sqrt(c * c + 1e-6) * w.astype(np.float64)
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)
    # unit weights: the output has mean square 1 / (1 + eps / ms)
    x = np.random.default_rng(9).standard_normal(hd).astype(np.float32) * 4
    y = oracle.qk_norm_row(x, np.ones(hd, np.float32), 1e-6).astype(np.float64)
    assert abs(np.mean(y * y) - 1.0) < 1e-5


def test_qk_norm_sits_before_rope_in_append_and_attend():
    """K is normalized before the rotation and quantization (codes equal those of appending the
    normalized K), q before its rotation (outputs equal attending with normalized q)."""
    rng = np.random.default_rng(41)
    n_kv, hd, n_head = 2, 64, 4
    table = oracle.rope_table(64, hd, 10000.0)
    wq = (rng.standard_normal(hd) * 0.3 + 1).astype(np.float32)
    wk = (rng.standard_normal(hd) * 0.3 + 1).astype(np.float32)
    k = rng.standard_normal((1, 20, n_kv, hd), dtype=np.float32) * 3
    v = rng.standard_normal((1, 20, n_kv, hd), dtype=np.float32)
    a = oracle.OracleKV(1, 64, n_kv, hd, table)
    a.k_norm, a.q_norm = wk, wq
    a.append(k, v)
    b = oracle.OracleKV(1, 64, n_kv, hd, table)
    kn = np.stack([[[oracle.qk_norm_row(k[0, t, h], wk) for h in range(n_kv)] for t in range(20)]])
    b.append(kn, v)
    assert np.array_equal(a.k_packed, b.k_packed) and np.array_equal(a.k_scale, b.k_scale)
    assert np.array_equal(a.v_packed, b.v_packed)
    q = rng.standard_normal((1, 20, n_head, hd), dtype=np.float32)
    qn = np.stack([[[oracle.qk_norm_row(q[0, t, h], wq) for h in range(n_head)] for t in range(20)]])
    np.testing.assert_array_equal(a.attend(q, 20), b.attend(qn, 20))


# ---- QKV projection (main_qkv, F16 weights) --------------------------------------------------

def test_f16_decode_every_bit_pattern():
    """f16_to_f32 (sh_layer_v1_int4.wgsl:7-34) over all 65536 patterns: IEEE half for every
    finite value (numpy's float16), 0 for inf and NaN as the shader returns."""
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert (got[~fin] == 0).all()


def test_project_exact_on_integers():
    """Small integers: every product and partial sum is exact in f32, so the dot is the
    integer matrix product (a transposed operand or a dropped term would show)."""
    rng = np.random.default_rng(1)
    x = rng.integers(-8, 9, size=(5, 192)).astype(np.float32)
    w = rng.integers(-8, 9, size=(7, 192)).astype(np.float16)
    got = oracle.project(x, w.view(np.uint16))
    ref = x.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(got, ref.astype(np.float32))


def test_project_sequential_f32_order():
    """The accumulation is one f32 sum in column order: against a float64 sum it is within the
    sequential-rounding bound, and it equals a numpy restatement of the same order exactly."""
    rng = np.random.default_rng(2)
    dim = 1024
    x = rng.standard_normal((3, dim)).astype(np.float32)
    w = (rng.standard_normal((4, dim)) * 0.05).astype(np.float16)
    got = oracle.project(x, w.view(np.uint16))
    wf = w.astype(np.float32)
    exact = x.astype(np.float64) @ wf.astype(np.float64).T
    bound = dim * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(wf).astype(np.float64).T)
    assert (np.abs(got - exact) <= bound).all()
    seq = np.zeros((3, 4), np.float32)
    for c in range(dim):            # order of the reference loop, one f32 rounding per step
        seq = (seq + (x[:, c:c + 1] * wf[None, :, c])).astype(np.float32)
    assert np.array_equal(got, seq)
    # a cancelling pair: order matters, and the oracle keeps the reference's
    xc = np.array([[1.0, 2.0 ** 24, -(2.0 ** 24)] + [0.0] * 61], np.float32)
    wc = np.zeros((1, 64), np.float16)
    wc[0, :3] = 1.0
    assert oracle.project(xc, wc.view(np.uint16))[0, 0] == 0.0   # (1 + 2^24) rounds to 2^24


def test_attn_proj_adds_the_projection_to_the_residual():
    """main_attn_proj: stash = the f32 dot, act = act + dot with one rounding (checked on exact
    integers, where the sum is the integer one, and against the projection itself)."""
    rng = np.random.default_rng(3)
    a = rng.integers(-4, 5, size=(3, 128)).astype(np.float32)
    w = rng.integers(-4, 5, size=(5, 128)).astype(np.float16)
    act = rng.integers(-100, 100, size=(3, 5)).astype(np.float32)
    out, stash = oracle.attn_proj(a, w.view(np.uint16), act)
    dot = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(stash, dot.astype(np.float32))
    assert np.array_equal(out, (act.astype(np.int64) + dot).astype(np.float32))
    af = rng.standard_normal((2, 256)).astype(np.float32)
    wf = (rng.standard_normal((3, 256)) * 0.1).astype(np.float16)
    actf = rng.standard_normal((2, 3)).astype(np.float32)
    out, stash = oracle.attn_proj(af, wf.view(np.uint16), actf)
    assert np.array_equal(stash, oracle.project(af, wf.view(np.uint16)))
    assert np.array_equal(out, (actf + stash).astype(np.float32))
