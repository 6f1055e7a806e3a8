"""GPU parity of the fused QK norm (Qwen3's apply_qk_norm, attention.rs:92-108, before RoPE):
K codes and scales bit-exact against the oracle with the norm on, and decode, fused decode and
prefill outputs within |err| <= 2e-3 + 1e-3*|ref|, for both decode kernels."""
import numpy as np
import pytest
import torch

from airframe_amd import TsError, synth
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu


def with_norm(p: Pair, rng, eps=1e-6, q=True, k=True):
    wq = (rng.standard_normal(p.hd) * 0.4 + 1.0).astype(np.float32) if q else None
    wk = (rng.standard_normal(p.hd) * 0.4 + 1.0).astype(np.float32) if k else None
    p.gpu.set_qk_norm(0, dev(wq) if q else None, dev(wk) if k else None, eps)
    p.ora.q_norm, p.ora.k_norm, p.ora.norm_eps = wq, wk, eps


def fill(p: Pair, rng, n, scale=None, step=512):
    done = 0
    while done < n:
        m = min(step, n - done)
        k = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd), scale)
        v = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd), scale)
        p.append(k, v)
        p.advance(m)
        done += m


def fused_step(p: Pair, rng, n_head, scale_kv=None, scale_q=None):
    k = synth.normal(rng, (p.n_seq, 1, p.n_kv, p.hd), scale_kv)
    v = synth.normal(rng, (p.n_seq, 1, p.n_kv, p.hd), scale_kv)
    q = synth.normal(rng, (p.n_seq, n_head, p.hd), scale_q)
    out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope).cpu().numpy()
    p.ora.append(k, v)
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    p.advance(1)
    return out, ref


@pytest.mark.parametrize("hd", [64, 128])
def test_append_codes_and_decode(gpu, hd):
    say(f"qk norm hd={hd}")
    rng = np.random.default_rng(400 + hd)
    p = Pair(3, 2, hd, 400, 1e6)
    with_norm(p, rng)
    fill(p, rng, 300, step=77)           # ragged chunks through the append kernel
    p.check_codes()
    for _ in range(2):
        out, ref = fused_step(p, rng, 8)  # fused append + decode
        assert_close(out, ref, "fused decode with QK norm")
    # separate append + decode
    k = synth.normal(rng, (3, 1, 2, hd))
    v = synth.normal(rng, (3, 1, 2, hd))
    q = synth.normal(rng, (3, 8, hd))
    p.append(k, v)
    out = p.gpu.attn_decode(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
    assert_close(out, ref, "decode with QK norm")
    p.advance(1)
    p.check_codes()


def test_prefill_with_norm_and_outliers(gpu):
    say("qk norm prefill")
    rng = np.random.default_rng(410)
    n_kv, n_head, hd = 8, 32, 128
    dims = synth.outlier_dims(n_kv, hd, 3)
    skv = synth.channel_scale(n_kv, n_kv, hd, dims)
    sq = synth.channel_scale(n_head, n_kv, hd, dims)
    p = Pair(2, n_kv, hd, 700, 1e6)
    with_norm(p, rng)
    fill(p, rng, 300, skv[None, None])
    k = synth.normal(rng, (2, 200, n_kv, hd), skv[None, None])
    v = synth.normal(rng, (2, 200, n_kv, hd), skv[None, None])
    q = synth.normal(rng, (2, 200, n_head, hd), sq[None, None])
    p.append(k, v)
    out = p.gpu.attn_prefill(0, dev(q), p.rope).cpu().numpy()
    ref = p.ora.attend(q, 200, threads=8)
    assert_close(out, ref, "prefill with QK norm")
    p.advance(200)
    p.check_codes()


def test_long_split_kernel_with_norm(gpu):
    """Splits of >= 4 windows per wave (4x4x4 QK kernel) with the norm on q only, then on K."""
    say("qk norm long splits")
    rng = np.random.default_rng(420)
    p = Pair(32, 8, 128, 4400, 1e6)
    with_norm(p, rng, k=False)
    fill(p, rng, 4300, step=1024)
    out, ref = fused_step(p, rng, 32)
    assert_close(out, ref, "long-split decode, q norm")
    with_norm(p, rng)
    out, ref = fused_step(p, rng, 32)
    assert_close(out, ref, "long-split decode, q and K norm")
    p.check_codes()


def test_norm_off_again_and_bad_args(gpu):
    say("qk norm off")
    rng = np.random.default_rng(430)
    p = Pair(1, 2, 64, 64, 1e4)
    with_norm(p, rng)
    fill(p, rng, 10)
    p.gpu.set_qk_norm(0, None, None)
    p.ora.q_norm = p.ora.k_norm = None
    fill(p, rng, 10)
    p.check_codes()
    with pytest.raises(ValueError):
        p.gpu.set_qk_norm(0, torch.zeros(63, device="cuda"), None)
    with pytest.raises(TsError):
        p.gpu.set_qk_norm(5, None, None)


@pytest.mark.parametrize("hd", [64, 128])
def test_norm_softcap_and_compaction_together(gpu, hd):
    """QK norm, the tanh softcap and a compacted window base at once: codes bit-exact, fused
    decode and prefill within tolerance."""
    say(f"qk norm + softcap + compaction hd={hd}")
    rng = np.random.default_rng(900 + hd)
    p = Pair(2, 2, hd, 600, 1e6, rope_n_pos=1200)
    with_norm(p, rng)
    fill(p, rng, 400, step=150)
    n = int(p.ora.lens[0])
    p.gpu.compact(4, 200, 0)
    p.ora.shift(0, 4, 200)
    p.ora.advance_window_base(0, 200)
    p.ora.lens[0] = n - 200
    fill(p, rng, 50, step=50)
    p.check_codes()
    k = synth.normal(rng, (2, 1, 2, hd))
    v = synth.normal(rng, (2, 1, 2, hd))
    q = synth.normal(rng, (2, 8, hd))
    out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope, softcap=30.0).cpu().numpy()
    p.ora.append(k, v)
    assert_close(out, p.ora.attend(q[:, None], 1, softcap=30.0, threads=8)[:, 0], "fused decode")
    p.advance(1)
    k = synth.normal(rng, (2, 12, 2, hd))
    v = synth.normal(rng, (2, 12, 2, hd))
    q = synth.normal(rng, (2, 12, 8, hd))
    p.append(k, v)
    out = p.gpu.attn_prefill(0, dev(q), p.rope, softcap=30.0).cpu().numpy()
    assert_close(out, p.ora.attend(q, 12, softcap=30.0, threads=8), "prefill")
    p.advance(12)
    p.check_codes()
