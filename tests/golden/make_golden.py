"""Writes the golden fixtures of this directory.

    python tests/golden/make_golden.py

reference_kat.json -- the inputs of the reference's four INT4 known-answer tests
    (src/backend/bindless/test_int4_parity.rs:304-585) written out as data, with the outputs
    those tests state literally (scales and words) and the bounds they assert.
oracle_small.npz -- a small seeded append + decode + prefill case run through the C oracle,
    cross-checked against the independent numpy restatement before it is written.  It pins
    the oracle against drift and gives the GPU tests a fixed expected output.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import np_oracle, oracle  # noqa: E402

SMALL = dict(seed=1234, n_seq=2, n_kv=2, n_head=4, hd=64, prefill=40, chunk=24, base=10000.0)


def f32list(x):
    return [float(v) for v in np.asarray(x, np.float32)]


def reference_kat():
    hd64 = np.arange(64, dtype=np.float32)
    ramp = (hd64 * np.float32(0.1) - np.float32(3.15)).astype(np.float32)          # :312-314
    sinus = (np.sin((hd64 * np.float32(0.3) - np.float32(9.5)).astype(np.float32)) * np.float32(2.5)).astype(np.float32)  # :316-318
    amps = [1.0, 2.0, 0.5, 7.0]                                                        # :411
    mh_k = [(np.float32(a) * ((hd64 / np.float32(64.0)) * np.float32(2.0) - np.float32(1.0))).astype(np.float32) for a in amps]  # :416-418
    mh_v = [(np.float32(a) * (hd64 * np.float32(0.1) - np.float32(3.15)) / np.float32(3.15)).astype(np.float32) for a in amps]  # :419-421
    alt = np.array([1000.0 if d % 2 == 0 else -1000.0 for d in range(8)], np.float32)  # :542-544
    return {
        "source": "src/backend/bindless/test_int4_parity.rs",
        "cases": [
            {"name": "zero_vector_no_nan", "lines": "489-520", "x": [0.0] * 8,
             "expect_scale": 1.0, "expect_words": [0x88888888]},
            {"name": "extreme_all_positive", "lines": "525-572", "x": [1000.0] * 8,
             "expect_words": [0xFFFFFFFF], "expect_scale_f32_of": "1000/7"},
            {"name": "extreme_alternating", "lines": "533-585", "x": f32list(alt),
             "roundtrip_bound": "scale/2 + 1.0"},
            {"name": "single_head_ramp_k", "lines": "306-392", "x": f32list(ramp),
             "expect_max_abs": 3.15, "roundtrip_bound": "scale/2 + 1e-5"},
            {"name": "single_head_sinusoid_v", "lines": "316-392", "x": f32list(sinus),
             "roundtrip_bound": "scale/2 + 1e-5"},
        ] + [
            {"name": f"multi_head_k_amp{a}", "lines": "397-485", "x": f32list(k),
             "expect_scale_close": float(np.float32(a) / np.float32(7.0)), "roundtrip_bound": "scale/2 + 1e-5"}
            for a, k in zip(amps, mh_k)
        ] + [
            {"name": f"multi_head_v_amp{a}", "lines": "397-485", "x": f32list(v),
             "roundtrip_bound": "scale/2 + 1e-5"}
            for a, v in zip(amps, mh_v)
        ],
    }


def oracle_small():
    c = SMALL
    rng = np.random.default_rng(c["seed"])
    n_seq, n_kv, n_head, hd = c["n_seq"], c["n_kv"], c["n_head"], c["hd"]
    P, C = c["prefill"], c["chunk"]
    max_seq = P + C + 1
    table = oracle.rope_table(max_seq, hd, c["base"])
    kv = oracle.OracleKV(n_seq, max_seq, n_kv, hd, table)
    k0 = rng.standard_normal((n_seq, P, n_kv, hd), dtype=np.float32)
    v0 = rng.standard_normal((n_seq, P, n_kv, hd), dtype=np.float32)
    kv.append(k0, v0)
    kv.advance(P)
    k1 = rng.standard_normal((n_seq, C, n_kv, hd), dtype=np.float32)
    v1 = rng.standard_normal((n_seq, C, n_kv, hd), dtype=np.float32)
    q1 = rng.standard_normal((n_seq, C, n_head, hd), dtype=np.float32)
    kv.append(k1, v1)
    o_prefill = kv.attend(q1, C)
    kv.advance(C)
    k2 = rng.standard_normal((n_seq, 1, n_kv, hd), dtype=np.float32)
    v2 = rng.standard_normal((n_seq, 1, n_kv, hd), dtype=np.float32)
    q2 = rng.standard_normal((n_seq, 1, n_head, hd), dtype=np.float32)
    kv.append(k2, v2)
    o_decode = kv.attend(q2, 1)

    # Cross-check against the independent numpy restatement before writing anything.
    n = max_seq
    for s in range(n_seq):
        kk = np.concatenate([k0[s], k1[s], k2[s]])
        vv = np.concatenate([v0[s], v1[s], v2[s]])
        cos, sin = table[:n, None, :, 0], table[:n, None, :, 1]
        kr = np_oracle.rotate(kk, cos, sin)
        ks, kw = np_oracle.quantize(kr)
        vs, vw = np_oracle.quantize(vv)
        assert (kw == kv.k_packed[s]).all() and (ks == kv.k_scale[s]).all()
        assert (vw == kv.v_packed[s]).all() and (vs == kv.v_scale[s]).all()
        kd, vd = np_oracle.dequantize(kw, ks), np_oracle.dequantize(vw, vs)
        qr = np_oracle.rotate(q1[s], table[P:P + C, None, :, 0], table[P:P + C, None, :, 1])
        ref = np_oracle.attend(qr, kd[:P + C], vd[:P + C], P)
        assert np.abs(ref - o_prefill[s]).max() < 1e-5
        qr = np_oracle.rotate(q2[s], table[P + C:P + C + 1, None, :, 0], table[P + C:P + C + 1, None, :, 1])
        ref = np_oracle.attend(qr, kd, vd, P + C)
        assert np.abs(ref - o_decode[s]).max() < 1e-5
    return dict(k0=k0, v0=v0, k1=k1, v1=v1, q1=q1, k2=k2, v2=v2, q2=q2,
                k_packed=kv.k_packed, v_packed=kv.v_packed, k_scale=kv.k_scale,
                v_scale=kv.v_scale, o_prefill=o_prefill, o_decode=o_decode,
                config=np.array(json.dumps(c)))


def main():
    with open(os.path.join(HERE, "reference_kat.json"), "w") as f:
        json.dump(reference_kat(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "oracle_small.npz"), **oracle_small())
    print("wrote reference_kat.json, oracle_small.npz")


if __name__ == "__main__":
    main()
