"""GPU parity of the split-K INT4 decode attention against the CPU oracle (attention.rs:236-313
over the dequantized INT4 cache), within |err| <= 2e-3 + 1e-3*|ref|, plus the codes of every
token appended on the way (bit-exact)."""
import json
import os

import numpy as np
import pytest
import torch

from airframe_amd import synth
from oracle import oracle
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def decode_step(p: Pair, rng, n_head, scale_kv=None, scale_q=None, softcap=0.0, check=True):
    n_seq, n_kv, hd = p.n_seq, p.n_kv, p.hd
    k = synth.normal(rng, (n_seq, 1, n_kv, hd), scale_kv)
    v = synth.normal(rng, (n_seq, 1, n_kv, hd), scale_kv)
    q = synth.normal(rng, (n_seq, n_head, hd), scale_q)
    p.append(k, v)
    out = p.gpu.attn_decode(0, dev(q), p.rope, softcap=softcap).cpu().numpy()
    ref = p.ora.attend(q[:, None], 1, softcap=softcap, threads=8)[:, 0] if check else None
    p.advance(1)
    return out, ref


def prefill_cache(p: Pair, rng, n, scale_kv=None, step=512):
    done = 0
    while done < n:
        m = min(step, n - done)
        k = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd), scale_kv)
        v = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd), scale_kv)
        p.append(k, v)
        p.advance(m)
        done += m


def test_config1_llama32_1b_single_layer(gpu):
    """32 q / 8 kv heads, hd 64, batch 1, 512 cached + 1 appended, theta 5e5."""
    say("decode cfg1")
    rng = np.random.default_rng(1)
    p = Pair(1, 8, 64, 513, 500000.0)
    prefill_cache(p, rng, 512)
    out, ref = decode_step(p, rng, 32)
    assert_close(out, ref, "cfg1 out")
    p.check_codes()


@pytest.mark.parametrize("hd,n_kv,G,ctx,softcap", [
    (64, 8, 4, 300, 0.0),     # 5 windows: one 8-wave workgroup per stream
    (64, 8, 4, 1000, 30.0),   # 16 windows: 16 waves
    (40, 2, 6, 700, 0.0),     # 40-dim rows stored as 64: 16 waves
    (128, 8, 3, 511, 0.0),    # 8 windows of 128-dim rows: 8 waves
    (96, 4, 8, 450, 30.0),    # 96-dim rows stored as 128
    (64, 8, 12, 600, 0.0),    # two head groups of the 16x16 kernel per kv head
])
def test_wide_no_split_plans(gpu, hd, n_kv, G, ctx, softcap):
    """Batch 1, 5-16 windows of context: one 8- or 16-wave workgroup per stream, no split and
    no combine launch.  The separate append + attention, the fused one, and the fused one that
    advances the lengths inside the kernel, each within tolerance; codes bit-exact."""
    say(f"decode wide hd={hd} n_kv={n_kv} G={G} ctx={ctx} softcap={softcap}")
    rng = np.random.default_rng(40 + ctx)
    n_head = n_kv * G
    p = Pair(1, n_kv, hd, ctx + 4, 500000.0)
    prefill_cache(p, rng, ctx)
    out, ref = decode_step(p, rng, n_head, softcap=softcap)
    assert_close(out, ref, "separate")
    for adv in (False, True):
        k = synth.normal(rng, (1, 1, n_kv, hd))
        v = synth.normal(rng, (1, 1, n_kv, hd))
        q = synth.normal(rng, (1, n_head, hd))
        out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope, softcap=softcap,
                                       advance=adv).cpu().numpy()
        p.ora.append(k, v)
        ref = p.ora.attend(q[:, None], 1, softcap=softcap, threads=8)[:, 0]
        if adv:
            p.ora.advance(1)
        else:
            p.advance(1)
        assert_close(out, ref, f"fused, advance={adv}")
    assert p.gpu.seq_lens() == [ctx + 3]
    p.check_codes()


@pytest.mark.parametrize("scale,yarn", [(0.25, (1.0, 32.0)), (0.5, (0.0, 0.0))])
def test_scaled_rope_tables(gpu, scale, yarn):
    """A YaRN (preflight.rs:77-97) and a linear (scale < 1, :88-90) table: the appended codes
    bit-exact and the decode within tolerance, both against the oracle on the same table."""
    say(f"decode rope scale={scale} yarn={yarn}")
    rng = np.random.default_rng(31)
    p = Pair(2, 4, 128, 1500, 500000.0, rope_n_pos=4096, rope_scale=scale, yarn=yarn)
    prefill_cache(p, rng, 1200)
    for _ in range(2):
        out, ref = decode_step(p, rng, 16)
        assert_close(out, ref, "scaled-rope out")
    p.check_codes()


def test_gqa3_hd128_llama32_3b_shape(gpu):
    """Config 2's head shape (24 q / 8 kv, group 3) at a shorter context, several steps."""
    say("decode gqa3")
    rng = np.random.default_rng(2)
    p = Pair(1, 8, 128, 800, 500000.0)
    prefill_cache(p, rng, 700)
    for _ in range(3):
        out, ref = decode_step(p, rng, 24)
        assert_close(out, ref, "gqa3 out")
    p.check_codes()


def test_tinyllama_shape_batch1(gpu):
    """TinyLlama-1.1B's attention (32 q / 4 kv heads, group 8, hd 64, theta 1e4), the model of the
    reference's own INT4 soak test, at batch 1 and ctx 2048: fused append + decode over several
    steps against the oracle, the cache bit-exact."""
    say("decode tinyllama shape")
    rng = np.random.default_rng(11)
    p = Pair(1, 4, 64, 2100, 10000.0)
    prefill_cache(p, rng, 2040)
    for _ in range(3):
        k = synth.normal(rng, (1, 1, 4, 64))
        v = synth.normal(rng, (1, 1, 4, 64))
        q = synth.normal(rng, (1, 32, 64))
        out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope).cpu().numpy()
        p.ora.append(k, v)
        ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
        p.advance(1)
        assert_close(out, ref, "tinyllama out")
    p.check_codes()


def test_batch_outliers_qwen3_shape(gpu):
    """Config 3's shape (32/8, hd 128, theta 1e6, x8 outlier channels on 2% of dims) at
    batch 4 and context 3000."""
    say("decode outliers")
    rng = np.random.default_rng(3)
    n_kv, n_head, hd = 8, 32, 128
    dims = synth.outlier_dims(n_kv, hd, 3)
    skv = synth.channel_scale(n_kv, n_kv, hd, dims)
    sq = synth.channel_scale(n_head, n_kv, hd, dims)
    p = Pair(4, n_kv, hd, 3100, 1e6)
    prefill_cache(p, rng, 3000, skv[None, None])
    for _ in range(2):
        out, ref = decode_step(p, rng, n_head, skv[None, None], sq[None])
        assert_close(out, ref, "outlier out")


def test_ragged_lengths_and_split_boundaries(gpu):
    """Per-sequence lengths around every window/split edge, including an empty cache."""
    say("decode ragged")
    rng = np.random.default_rng(4)
    lens = [0, 1, 31, 63, 64, 65, 127, 128, 255, 256, 257, 1000, 1087, 1088, 1089, 2047]
    n_seq, n_kv, hd = len(lens), 2, 128
    p = Pair(n_seq, n_kv, hd, 2100, 1e6)
    # fill each sequence to its own length: fill all to max, then cut lengths back
    prefill_cache(p, rng, max(lens))
    p.set_lens(lens)
    for _ in range(2):
        out, ref = decode_step(p, rng, 8)
        assert_close(out, ref, "ragged out")
    p.check_codes()


def test_softcap(gpu):
    say("decode softcap")
    rng = np.random.default_rng(5)
    p = Pair(2, 4, 64, 400, 10000.0)
    prefill_cache(p, rng, 300, np.float32(3.0))
    out, ref = decode_step(p, rng, 16, np.float32(3.0), np.float32(3.0), softcap=5.0)
    assert_close(out, ref, "softcap out")


def test_group8_and_group1(gpu):
    say("decode group 8 / 1")
    rng = np.random.default_rng(6)
    for n_kv, n_head in ((2, 16), (4, 4)):
        p = Pair(2, n_kv, 128, 600, 500000.0)
        prefill_cache(p, rng, 513)
        out, ref = decode_step(p, rng, n_head)
        assert_close(out, ref, f"G={n_head // n_kv} out")


def test_golden_fixture_through_gpu(gpu):
    """tests/golden/oracle_small.npz: append 40, chunk 24 (prefill kernel), decode 1."""
    say("golden fixture")
    g = np.load(os.path.join(GOLD, "oracle_small.npz"))
    c = json.loads(str(g["config"]))
    P, C = c["prefill"], c["chunk"]
    p = Pair(c["n_seq"], c["n_kv"], c["hd"], P + C + 1, c["base"])
    p.gpu.append_quant(0, dev(g["k0"]), dev(g["v0"]), p.rope)
    p.gpu.increment(P)
    p.gpu.append_quant(0, dev(g["k1"]), dev(g["v1"]), p.rope)
    o1 = p.gpu.attn_prefill(0, dev(g["q1"]), p.rope).cpu().numpy()
    assert_close(o1, g["o_prefill"], "golden prefill")
    p.gpu.increment(C)
    p.gpu.append_quant(0, dev(g["k2"]), dev(g["v2"]), p.rope)
    o2 = p.gpu.attn_decode(0, dev(g["q2"][:, 0]), p.rope).cpu().numpy()
    assert_close(o2, g["o_decode"][:, 0], "golden decode")
    torch.cuda.synchronize()
    for s in range(c["n_seq"]):
        kp, vp, ks, vs = p.gpu.export(0, s, 0, P + C + 1)
        assert np.array_equal(kp.cpu().numpy().view(np.uint32), g["k_packed"][s])
        assert np.array_equal(vp.cpu().numpy().view(np.uint32), g["v_packed"][s])
        assert np.array_equal(ks.cpu().numpy(), g["k_scale"][s])
        assert np.array_equal(vs.cpu().numpy(), g["v_scale"][s])


ORACLE_THREADS = min(16, os.cpu_count() or 1)  # the GPU box's CPU share


def _full_size(n_seq, n_kv, n_head, hd, lens, base, seed, outliers, fused=False, softcap=0.0, norm=False):
    """One layer at the full BASELINE shape: the GPU runs every sequence and the oracle checks
    every (sequence, head) output on identical inputs (generated on the device and copied
    back), and every packed word and scale of the cache bit-exact.  With `fused`, the new
    token goes through ts_attn_decode_append (the launch bench.py times), otherwise through
    ts_append_quant then ts_attn_decode.  `softcap`: Gemma-2's score cap; `norm`: Qwen3's QK
    norm with random weights."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    dims = synth.outlier_dims(n_kv, hd, seed) if outliers else None
    skv = torch.as_tensor(synth.channel_scale(n_kv, n_kv, hd, dims)).cuda()
    sq = torch.as_tensor(synth.channel_scale(n_head, n_kv, hd, dims)).cuda()
    max_len = max(lens)
    p = Pair(n_seq, n_kv, hd, max_len + 1, base)
    if norm:
        wrng = np.random.default_rng(seed)
        wq = (wrng.standard_normal(hd) * 0.4 + 1.0).astype(np.float32)
        wk = (wrng.standard_normal(hd) * 0.4 + 1.0).astype(np.float32)
        p.gpu.set_qk_norm(0, dev(wq), dev(wk), 1e-6)
        p.ora.q_norm, p.ora.k_norm, p.ora.norm_eps = wq, wk, 1e-6
    step = 2048
    for t0 in range(0, max_len, step):
        m = min(step, max_len - t0)
        k = torch.randn((n_seq, m, n_kv, hd), generator=gen, device="cuda") * skv
        v = torch.randn((n_seq, m, n_kv, hd), generator=gen, device="cuda") * skv
        p.gpu.append_quant(0, k, v, p.rope)
        p.ora.append(k.cpu().numpy(), v.cpu().numpy())
        p.advance(m)
    p.set_lens(lens)
    k1 = torch.randn((n_seq, 1, n_kv, hd), generator=gen, device="cuda") * skv
    v1 = torch.randn((n_seq, 1, n_kv, hd), generator=gen, device="cuda") * skv
    q = torch.randn((n_seq, n_head, hd), generator=gen, device="cuda") * sq
    if fused:
        out = p.gpu.attn_decode_append(0, k1, v1, q, p.rope, softcap=softcap).cpu().numpy()
    else:
        p.gpu.append_quant(0, k1, v1, p.rope)
        out = p.gpu.attn_decode(0, q, p.rope, softcap=softcap).cpu().numpy()
    p.ora.append(k1.cpu().numpy(), v1.cpu().numpy())
    ref = p.ora.attend(q.cpu().numpy()[:, None], 1, softcap=softcap, threads=ORACLE_THREADS)[:, 0]
    assert_close(out, ref, f"full-size decode, every sequence and head (lens {min(lens)}..{max(lens)})")
    # the whole cache, the appended row included
    p.check_codes(upto=[l + 1 for l in lens])


def test_full_size_config3_one_layer(gpu):
    """Config 3 at full size (batch 32, ctx 8192, outliers), one layer, every head."""
    say("decode full cfg3")
    _full_size(32, 8, 32, 128, [8192] * 32, 1e6, 33, True)


def test_full_size_config3_fused(gpu):
    """Config 3 at full size through the fused append + decode launch that bench.py times:
    every head against the oracle, the whole cache (appended row included) bit-exact."""
    say("decode full cfg3 fused")
    _full_size(32, 8, 32, 128, [8192] * 32, 1e6, 34, True, fused=True)


def test_full_size_config4_ragged_fused(gpu):
    """Config 4 (ragged 16K-32K, batch 8) through the fused launch."""
    say("decode full cfg4 fused")
    rng = np.random.default_rng(45)
    lens = [int(x) for x in rng.integers(16384, 32768, size=8)]
    _full_size(8, 8, 32, 128, lens, 500000.0, 45, False, fused=True)


def test_full_size_config4_ragged_one_layer(gpu):
    """Config 4 at full size: batch 8, lengths ~U[16K, 32K] (seeded), one layer."""
    say("decode full cfg4")
    rng = np.random.default_rng(44)
    lens = [int(x) for x in rng.integers(16384, 32768, size=8)]
    _full_size(8, 8, 32, 128, lens, 500000.0, 44, False)


def test_full_size_config2_fused(gpu):
    """Config 2's decode step at its largest context (batch 1, 24/8 heads, hd 128, 4352 cached
    + 1 appended) through the fused launch bench.py times for config 2."""
    say("decode full cfg2 fused")
    _full_size(1, 8, 24, 128, [4352], 500000.0, 23, False, fused=True)


def test_config2_batch1_long_context(gpu):
    """Config 2's decode shape at its full context (batch 1, 24/8 heads, hd 128, 4352 keys):
    one sequence spread over many splits, so the split merge carries the result."""
    say("decode cfg2 full context")
    rng = np.random.default_rng(22)
    p = Pair(1, 8, 128, 4353, 500000.0)
    prefill_cache(p, rng, 4351, step=1024)
    for _ in range(2):
        k = synth.normal(rng, (1, 1, 8, 128))
        v = synth.normal(rng, (1, 1, 8, 128))
        q = synth.normal(rng, (1, 24, 128))
        p.append(k, v)
        out = p.gpu.attn_decode(0, dev(q), p.rope)
        ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
        assert_close(out.cpu().numpy(), ref, "cfg2 out")
        p.advance(1)


@pytest.mark.parametrize("hd,n_kv,n_head,n_seq,ctx,fused", [
    (256, 8, 16, 4, 8192, True),    # Gemma-2-9B's attention shape: 256-dim rows, 2 q heads per kv head
    (256, 4, 16, 4, 16000, False),  # 4 q heads per kv head, no append
    (96, 8, 32, 4, 8000, True),     # padded: stored as 128 dims
    (200, 4, 16, 8, 8192, True),    # padded: stored as 256 dims
    # two halves of 4 query heads (G 5..8)
    (128, 8, 64, 8, 8192, True),    # Llama-3-70B's attention shape: G = 8
    (128, 4, 28, 8, 8192, False),   # Qwen2.5-7B's: G = 7
    (64, 8, 40, 8, 8192, True),     # G = 5 on 64-dim rows
    (64, 8, 32, 8, 8192, False),    # Llama-3.2-1B's attention shape at batch 8: G = 4, 64-dim rows
    (256, 4, 24, 8, 8192, True),    # G = 6 on 256-dim rows
    (96, 8, 48, 8, 8000, True),     # G = 6, padded: stored as 128 dims
    # four halves (G 9..16)
    (128, 8, 128, 8, 8192, True),   # Llama-3.1-405B's attention shape: G = 16
    (64, 4, 48, 8, 8192, False),    # G = 12 on 64-dim rows (two head groups of waves)
    (64, 8, 128, 8, 8192, True),    # G = 16 on 64-dim rows
    (96, 8, 80, 8, 8000, True),     # G = 10, padded: stored as 128 dims
    # one kv head (Gemma-2B's 8 q / 1 kv): few streams, ~7 splits per sequence and the combine
    (128, 1, 8, 32, 8192, True),
    (128, 1, 16, 32, 8192, False),
])
def test_integer_kernel_wide_and_padded_rows(gpu, hd, n_kv, n_head, n_seq, ctx, fused):
    """The integer-QK kernel on 64-, 128-, 256-dim and padded rows with 2..16 query heads per kv
    head, at contexts whose plan gives every wave >= 4 windows (so this kernel runs): every
    head against the oracle, the whole cache bit-exact."""
    say(f"decode integer kernel hd={hd} G={n_head // n_kv} ctx={ctx} fused={fused}")
    rng = np.random.default_rng(hd + ctx)
    lens = [int(x) for x in rng.integers(ctx - 300, ctx, size=n_seq)]
    _full_size(n_seq, n_kv, n_head, hd, lens, 10000.0, hd + n_head, False, fused=fused)


@pytest.mark.parametrize("G,softcap,norm,hd", [(8, 30.0, False, 128), (8, 0.0, True, 128), (6, 50.0, True, 128),
                                                (3, 30.0, True, 128), (16, 30.0, True, 128), (13, 0.0, True, 128),
                                                (16, 30.0, True, 64), (7, 0.0, True, 64)])
def test_integer_kernel_softcap_and_qk_norm(gpu, G, softcap, norm, hd):
    """The integer-QK kernel with Gemma-2's score cap and Qwen3's QK norm, one, two or four
    halves of query heads (on 64-dim rows also two head groups of waves), fused append: every
    head against the oracle, the cache bit-exact."""
    say(f"decode integer kernel G={G} hd={hd} softcap={softcap} norm={norm}")
    rng = np.random.default_rng(G * 7 + int(softcap) + hd)
    lens = [int(x) for x in rng.integers(7800, 8192, size=8)]
    _full_size(8, 8, 8 * G, hd, lens, 1e6, 50 + G, True, fused=True, softcap=softcap, norm=norm)


def test_one_long_sequence_among_many_short(gpu):
    """More (sequence, kv head) streams than the plan's workgroup target, one sequence far
    longer than the rest: the plan still splits that one (its splits merge in the combine);
    every head against the oracle, the cache bit-exact."""
    say("decode one long sequence among 31 short")
    rng = np.random.default_rng(77)
    lens = [20000] + [int(x) for x in rng.integers(64, 400, size=31)]
    _full_size(32, 8, 32, 128, lens, 1e6, 78, False, fused=True)


def test_misaligned_buffers_rejected(gpu):
    """Device arrays must be 16-byte aligned: a misaligned workspace, q or out is refused
    before anything is launched."""
    say("decode misaligned buffers")
    from airframe_amd._lib import TsError
    p = Pair(1, 2, 64, 2048, 10000.0)
    prefill_cache(p, np.random.default_rng(7), 1500)
    k = synth.normal(np.random.default_rng(8), (1, 1, 2, 64))
    p.gpu.append_quant(0, dev(k), dev(k), p.rope)
    ws = p.gpu.workspace(8)
    buf = torch.empty(ws.numel() + 16, dtype=torch.uint8, device="cuda")
    q = torch.zeros((1, 8, 64), device="cuda")
    with pytest.raises(TsError):
        p.gpu.attn_decode(0, q, p.rope, workspace=buf[4:4 + ws.numel()])
    flat = torch.zeros(8 * 64 + 4, device="cuda")
    with pytest.raises(TsError):
        p.gpu.attn_decode(0, flat[1:1 + 8 * 64].view(1, 8, 64), p.rope)
    with pytest.raises(TsError):
        p.gpu.attn_decode(0, q, p.rope, out=flat[2:2 + 8 * 64].view(1, 8, 64))
    with pytest.raises(TsError):
        p.gpu.append_quant(0, flat[1:1 + 2 * 64].view(1, 1, 2, 64), dev(k), p.rope)
    p.gpu.attn_decode(0, q, p.rope, workspace=buf[16:16 + ws.numel()])
    torch.cuda.synchronize()
