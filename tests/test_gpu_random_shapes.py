"""Seeded random shapes through the whole cache lifecycle, against the oracle: ragged lengths,
a prefill chunk at every sequence's own length, then decode steps alternating the fused
append + attention (the last one advancing the lengths inside its launch) with the separate
append and attention.  The head dim, group size, kv heads, batch, lengths, softcap and QK norm
are drawn per case from what the path supports (head dims that are multiples of 8 up to 256,
any group size), so plan and kernel choices the fixed-shape tests do not pick get exercised.
INT4 codes and scales bit-exact after every step, outputs within 2e-3 + 1e-3 |ref|."""
import os

import numpy as np
import pytest

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def draw(seed):
    rng = np.random.default_rng(9000 + seed)
    hd = int(rng.choice([40, 64, 96, 128, 136, 192, 256]))
    n_kv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    n_seq = int(rng.integers(1, 5))
    fill = int(np.exp(rng.uniform(0.0, np.log(6000.0))))  # up to 6K: split plans too
    lens = [int(x) for x in rng.integers(0, fill + 1, size=n_seq)]
    chunk = int(rng.integers(1, 65))
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    norm = bool(rng.integers(0, 4) == 0)
    return rng, dict(hd=hd, n_kv=n_kv, G=G, n_seq=n_seq, fill=fill, lens=lens, chunk=chunk,
                     softcap=softcap, norm=norm)


@pytest.mark.parametrize("seed", range(40))
def test_random_shape_lifecycle(gpu, seed):
    rng, c = draw(seed)
    say(f"random shape seed={seed} {c}")
    hd, n_kv, n_seq, G = c["hd"], c["n_kv"], c["n_seq"], c["G"]
    n_head = n_kv * G
    steps = 3
    P = c["fill"] + c["chunk"] + steps + 1
    p = Pair(n_seq, n_kv, hd, P, float(rng.choice([1e4, 5e5, 1e6])))
    if c["norm"]:
        wq = (rng.standard_normal(hd) * 0.4 + 1.0).astype(np.float32)
        wk = (rng.standard_normal(hd) * 0.4 + 1.0).astype(np.float32)
        p.gpu.set_qk_norm(0, dev(wq), dev(wk), 1e-6)
        p.ora.q_norm, p.ora.k_norm, p.ora.norm_eps = wq, wk, 1e-6
    # the whole window filled, then each sequence cut back to its own length
    k = synth.normal(rng, (n_seq, c["fill"], n_kv, hd))
    v = synth.normal(rng, (n_seq, c["fill"], n_kv, hd))
    p.append(k, v)
    p.set_lens(c["lens"])
    # a prefill chunk at every sequence's own length
    T = c["chunk"]
    k = synth.normal(rng, (n_seq, T, n_kv, hd))
    v = synth.normal(rng, (n_seq, T, n_kv, hd))
    q = synth.normal(rng, (n_seq, T, n_head, hd))
    p.append(k, v)
    out = p.gpu.attn_prefill(0, dev(q), p.rope, softcap=c["softcap"]).cpu().numpy()
    ref = p.ora.attend(q, T, softcap=c["softcap"], threads=THREADS)
    assert_close(out, ref, f"prefill of {T} tokens")
    p.advance(T)
    p.check_codes()
    # decode steps
    for t in range(steps):
        k = synth.normal(rng, (n_seq, 1, n_kv, hd))
        v = synth.normal(rng, (n_seq, 1, n_kv, hd))
        q = synth.normal(rng, (n_seq, n_head, hd))
        if t % 2 == 0:
            last = t == steps - 1
            out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope, softcap=c["softcap"],
                                           advance=last).cpu().numpy()
            p.ora.append(k, v)
            ref = p.ora.attend(q[:, None], 1, softcap=c["softcap"], threads=THREADS)[:, 0]
            if last:
                p.ora.advance(1)  # the launch advanced the device and host lengths
            else:
                p.advance(1)
        else:
            p.append(k, v)
            out = p.gpu.attn_decode(0, dev(q), p.rope, softcap=c["softcap"]).cpu().numpy()
            ref = p.ora.attend(q[:, None], 1, softcap=c["softcap"], threads=THREADS)[:, 0]
            p.advance(1)
        assert_close(out, ref, f"decode step {t} ({'fused' if t % 2 == 0 else 'separate'})")
    assert p.gpu.seq_lens() == [int(x) for x in p.ora.lens]
    p.check_codes()
