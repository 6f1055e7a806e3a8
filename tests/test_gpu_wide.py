"""GPU parity beyond the configurations' shapes: GQA groups of more than 8 query heads per kv
head (the decode runs them as groups of 8, each reading the kv head's stream; the reference
accepts any n_head that n_head_kv divides, kv_cache.rs / attention.rs).  Decode (fused with
the append, and separate, with splits) and prefill against the oracle, |err| <= 2e-3 +
1e-3*|ref|; appended codes bit-exact."""
import numpy as np
import pytest

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say
from tests.test_gpu_decode_append import fill, fused_step
from tests.test_gpu_prefill import run_chunks

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_kv,n_head,hd,softcap", [
    (2, 24, 128, 0.0),   # G = 12: a group of 8 and one of 4
    (1, 16, 64, 0.0),    # G = 16, one kv head
    (1, 32, 128, 30.0),  # G = 32 (multi-query), softcap
])
def test_fused_decode_large_groups(gpu, n_kv, n_head, hd, softcap):
    say(f"fused decode G={n_head // n_kv} n_kv={n_kv} hd={hd} softcap={softcap}")
    rng = np.random.default_rng(300 + n_head + hd)
    lens = [1500, 3, 640, 2047]
    p = Pair(len(lens), n_kv, hd, 2100, 500000.0)
    fill(p, rng, max(lens))
    p.set_lens(lens)
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head, softcap=softcap)
        assert_close(out, ref, "fused out")
    p.check_codes()


def test_separate_decode_large_group(gpu):
    say("separate decode G=12")
    rng = np.random.default_rng(310)
    n_kv, n_head, hd = 2, 24, 128
    p = Pair(3, n_kv, hd, 1300, 500000.0)
    fill(p, rng, 1200)
    p.set_lens([1200, 17, 800])
    k = synth.normal(rng, (3, 1, n_kv, hd))
    v = synth.normal(rng, (3, 1, n_kv, hd))
    q = synth.normal(rng, (3, n_head, hd))
    p.append(k, v)
    out = p.gpu.attn_decode(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    assert_close(out, ref, "decode out")


@pytest.mark.parametrize("n_kv,n_head,hd", [(2, 24, 128), (1, 16, 64)])
def test_prefill_large_groups(gpu, n_kv, n_head, hd):
    say(f"prefill G={n_head // n_kv} hd={hd}")
    rng = np.random.default_rng(320 + n_head)
    p = Pair(2, n_kv, hd, 300, 500000.0)
    p.set_lens([0, 37])
    run_chunks(p, rng, n_head, [50, 90])
    p.check_codes()


# ---- head dims other than 64 and 128 (stored padded to 64 / 128 dims) --------------------------

from tests import test_gpu_compaction as comp  # noqa: E402
from tests.test_gpu_qk_norm import with_norm  # noqa: E402


@pytest.mark.parametrize("hd,n_kv,n_head,rope_dim", [
    (96, 2, 8, None),    # Phi-3 style, stored as 128
    (80, 4, 16, 64),     # partial rotation, stored as 128
    (40, 2, 4, None),    # stored as 64, G <= 4
    (8, 1, 3, None),     # the smallest head dim the reference accepts
    (120, 1, 12, None),  # G = 12 with a padded head
    (256, 2, 4, None),   # Gemma-2 / Gemma-3 head dim
    (192, 1, 4, 128),    # stored as 256, partial rotation
    (136, 2, 16, None),  # just past 128: stored as 256, G = 8
])
def test_head_dims_append_decode_prefill(gpu, hd, n_kv, n_head, rope_dim):
    say(f"head_dim {hd} n_kv={n_kv} n_head={n_head} rope_dim={rope_dim}")
    rng = np.random.default_rng(500 + hd)
    p = Pair(3, n_kv, hd, 1400, 10000.0, rope_dim=rope_dim)
    fill(p, rng, 1100, step=300)  # ragged chunks through the append kernel
    p.set_lens([1100, 5, 700])
    p.check_codes()
    for _ in range(2):
        out, ref = fused_step(p, rng, n_head)
        assert_close(out, ref, f"hd {hd} fused decode")
    k = synth.normal(rng, (3, 1, n_kv, hd))
    v = synth.normal(rng, (3, 1, n_kv, hd))
    q = synth.normal(rng, (3, n_head, hd))
    p.append(k, v)
    out = p.gpu.attn_decode(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    assert_close(out, ref, f"hd {hd} decode")
    p.advance(1)
    run_chunks(p, rng, n_head, [33])
    p.check_codes()


@pytest.mark.parametrize("hd", [96, 48, 256])
def test_head_dims_qk_norm_and_compaction(gpu, hd):
    say(f"head_dim {hd}: qk norm, compaction")
    rng = np.random.default_rng(600 + hd)
    n_head = 8
    p = Pair(2, 2, hd, 400, 10000.0, rope_n_pos=1400)
    with_norm(p, rng)
    comp.fill(p, rng, 300)
    p.set_lens([300, 250])
    p.check_codes()
    comp.compact(p, 0, 4, 100)
    comp.compact(p, 1, 4, 37)
    p.check_codes()
    for _ in range(2):
        out, ref = comp.fused_step(p, rng, n_head)
        assert_close(out, ref, f"hd {hd} fused decode after compaction, qk norm")
    out, ref = comp.prefill_chunk(p, rng, n_head, 17)
    assert_close(out, ref, f"hd {hd} prefill after compaction, qk norm")
    p.check_codes()


def test_head_dim_256_softcap_long_splits(gpu):
    """Gemma-2's attention shape (head dim 256, two query heads per kv head, logit softcap 50)
    with contexts long enough for several splits per sequence."""
    say("head_dim 256 softcap, splits")
    rng = np.random.default_rng(700)
    p = Pair(2, 4, 256, 4200, 10000.0)
    fill(p, rng, 4000, step=1000)
    p.set_lens([4000, 2500])
    for _ in range(2):
        out, ref = fused_step(p, rng, 8, softcap=50.0)
        assert_close(out, ref, "hd 256 fused decode, softcap")
    p.check_codes(upto=[p.ora.lens[0], p.ora.lens[1]])
