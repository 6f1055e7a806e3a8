"""GPU parity of the fused QKV projection + INT4 append (main_qkv, sh_layer_v1_int4.wgsl:454-575,
F16 weights, followed by quantize_kv).

* q and the raw K/V projections against the oracle's f32 dot (or_project) within
  |err| <= 2e-3 + 1e-3*|ref|;
* the cache codes and scales bit-exact against the oracle's append of the K/V projections the
  kernel itself produced (the epilogue is the append's arithmetic, so from the same f32 input
  it must write the same bits);
* a run without the raw K/V outputs writes the same cache and q bits.
Shapes cover the decode rows (one token per sequence, > 32 sequences), block rows (prefill
chunks from ragged, unaligned lengths, in 32- and 64-row tiles), the reduction split over dim
and the unsplit one,
an odd number of query or kv heads, head_dim 128 and 64, the QK norm and a compacted
sequence."""
import numpy as np
import pytest
import torch

from airframe_amd import TsError
from airframe_amd.kv_cache import KVCache
from tests.gpu_util import Pair, assert_close, dev, say
from oracle import oracle

pytestmark = pytest.mark.gpu


def weights(rng, rows, dim, scale=0.02):
    w = (rng.standard_normal((rows, dim)) * scale).astype(np.float16)
    return w, w.view(np.uint16)


def run_case(p: Pair, rng, n_tok, dim, n_head, x_scale=1.0):
    hd, n_kv, n_seq = p.hd, p.n_kv, p.n_seq
    wq, wq_b = weights(rng, n_head * hd, dim)
    wk, wk_b = weights(rng, n_kv * hd, dim)
    wv, wv_b = weights(rng, n_kv * hd, dim)
    x = (rng.standard_normal((n_seq, n_tok, dim)) * x_scale).astype(np.float32)
    k_out = torch.empty((n_seq, n_tok, n_kv, hd), dtype=torch.float32, device="cuda")
    v_out = torch.empty_like(k_out)
    q = p.gpu.qkv_append(0, dev(x), dev(wq), dev(wk), dev(wv), p.rope, kv_out=(k_out, v_out))
    torch.cuda.synchronize()
    q, k_out, v_out = q.cpu().numpy(), k_out.cpu().numpy(), v_out.cpu().numpy()

    xf = x.reshape(-1, dim)
    assert_close(q.reshape(n_seq * n_tok, -1), oracle.project(xf, wq_b), "q projection")
    assert_close(k_out.reshape(n_seq * n_tok, -1), oracle.project(xf, wk_b), "k projection")
    assert_close(v_out.reshape(n_seq * n_tok, -1), oracle.project(xf, wv_b), "v projection")

    # the cache holds exactly what the append would have made of those projections
    p.ora.append(k_out, v_out)
    lens_before = p.ora.lens.copy()
    p.advance(n_tok)
    p.check_codes()
    return x, (wq, wk, wv), q, lens_before


@pytest.mark.parametrize("n_seq,n_tok,dim,n_head,n_kv", [
    (40, 1, 2048, 16, 4),    # decode rows, two row tiles, split reduction
    (32, 1, 4096, 32, 8),    # Qwen3-8B / Llama-3-8B projection shape, decode batch 32
    (3, 1, 256, 8, 2),       # decode rows, no split
    (3, 70, 1024, 8, 2),     # block rows, split
    (3, 70, 256, 8, 2),      # block rows, no split
    (2, 33, 512, 3, 1),      # odd query-head count: the last q tile is half empty
    (4, 300, 256, 32, 8),    # prefill chunks: 64-row tiles (two V blocks per workgroup)
    (70, 1, 320, 8, 2),      # decode rows in 64-row tiles (dim not a multiple of 256: no split)
])
def test_qkv_append(gpu, n_seq, n_tok, dim, n_head, n_kv):
    say(f"qkv n_seq={n_seq} n_tok={n_tok} dim={dim} n_head={n_head} n_kv={n_kv}")
    rng = np.random.default_rng(dim + n_tok + n_seq)
    max_seq = 128 + 2 * n_tok + 16
    p = Pair(n_seq, n_kv, 128, max_seq, 1e6)
    lens = rng.integers(0, 100, size=n_seq).astype(np.int32)
    lens[0] = 0
    p.set_lens(lens)
    x, (wq, wk, wv), q, lens_before = run_case(p, rng, n_tok, dim, n_head)

    if n_tok > 1:  # a second chunk continuing where the first ended
        run_case(p, rng, 5, dim, n_head)

    # the same call without the raw K/V outputs: identical q and cache bits
    g2 = KVCache.new_int4(1, n_kv, 128, max_seq, n_seq)
    for s, l in enumerate(lens_before):
        g2.set_seq_len(int(l), seq=s)
    q2 = g2.qkv_append(0, dev(x), dev(wq), dev(wk), dev(wv), p.rope).cpu().numpy()
    assert np.array_equal(q2.view(np.uint32), q.view(np.uint32))
    torch.cuda.synchronize()
    for s in range(n_seq):
        a = [t.cpu() for t in p.gpu.export(0, s, int(lens_before[s]), n_tok)]
        b = [t.cpu() for t in g2.export(0, s, int(lens_before[s]), n_tok)]
        for u, w in zip(a, b):
            assert torch.equal(u.view(torch.uint8), w.view(torch.uint8))


def test_qkv_append_qk_norm_and_compaction(gpu):
    say("qkv with QK norm after a compaction")
    rng = np.random.default_rng(77)
    n_seq, n_kv, n_head, dim = 2, 2, 8, 512
    p = Pair(n_seq, n_kv, 128, 512, 1e6, rope_n_pos=1024)
    wq_n = (rng.standard_normal(128) * 0.4 + 1.0).astype(np.float32)
    wk_n = (rng.standard_normal(128) * 0.4 + 1.0).astype(np.float32)
    p.gpu.set_qk_norm(0, dev(wq_n), dev(wk_n), 1e-6)
    p.ora.q_norm, p.ora.k_norm, p.ora.norm_eps = wq_n, wk_n, 1e-6
    run_case(p, rng, 200, dim, n_head)          # prefill blocks with the norm
    # compact sequence 1 (sinks 4, shift 120) on both sides, then continue
    n = int(p.ora.lens[1])
    p.gpu.compact(4, 120, 1)
    p.ora.shift(1, 4, 120)
    p.ora.advance_window_base(1, 120)
    p.ora.lens[1] = n - 120
    run_case(p, rng, 1, dim, n_head)            # decode rows, rotated past the window base
    run_case(p, rng, 40, dim, n_head)           # block rows, rotated past the window base


def test_qkv_append_errors(gpu):
    say("qkv errors")
    rng = np.random.default_rng(5)
    p = Pair(2, 2, 128, 64, 1e4)
    wq, _ = weights(rng, 8 * 128, 256)
    wk, _ = weights(rng, 2 * 128, 256)
    x = dev(np.zeros((2, 1, 256), np.float32))
    with pytest.raises(ValueError):            # wrong weight shape
        p.gpu.qkv_append(0, x, dev(wq), dev(wq), dev(wk), p.rope)
    x100 = dev(np.zeros((2, 1, 100), np.float32))
    w100 = dev(np.zeros((8 * 128, 100), np.float16))
    k100 = dev(np.zeros((2 * 128, 100), np.float16))
    with pytest.raises(TsError) as e:          # dim not a multiple of 64
        p.gpu.qkv_append(0, x100, w100, k100, k100, p.rope)
    assert e.value.code == -1
    with pytest.raises(TsError) as e:          # too small a workspace for a split reduction
        xs = dev(np.zeros((2, 1, 4096), np.float32))
        ws = torch.empty(16, dtype=torch.uint8, device="cuda")
        p.gpu.qkv_append(0, xs, dev(np.zeros((1024, 4096), np.float16)),
                         dev(np.zeros((256, 4096), np.float16)), dev(np.zeros((256, 4096), np.float16)),
                         p.rope, workspace=ws)
    assert e.value.code == -6
    p.gpu.set_seq_len(60, seq=0)
    with pytest.raises(TsError) as e:          # past max_seq
        p.gpu.qkv_append(0, dev(np.zeros((2, 8, 256), np.float32)), dev(wq), dev(wk), dev(wk), p.rope)
    assert e.value.code == -2


@pytest.mark.parametrize("n_seq,n_tok,dim,n_head,n_kv", [
    (5, 1, 2048, 32, 8),     # Llama-3.2-1B projection shape, decode rows, split reduction
    (3, 70, 512, 8, 2),      # block rows, split
    (4, 300, 256, 32, 8),    # prefill chunks in 64-row tiles
    (70, 1, 320, 6, 3),      # odd kv-head count: the last (K, V) tile holds one pair
])
def test_qkv_append_hd64(gpu, n_seq, n_tok, dim, n_head, n_kv):
    say(f"qkv hd64 n_seq={n_seq} n_tok={n_tok} dim={dim} n_head={n_head} n_kv={n_kv}")
    rng = np.random.default_rng(640 + dim + n_tok)
    p = Pair(n_seq, n_kv, 64, 128 + 2 * n_tok + 16, 5e5)
    lens = rng.integers(0, 100, size=n_seq).astype(np.int32)
    p.set_lens(lens)
    run_case(p, rng, n_tok, dim, n_head)
    run_case(p, rng, 3, dim, n_head)


@pytest.mark.parametrize("hd,n_seq,n_tok,dim,n_head,n_kv", [
    (96, 4, 1, 1024, 8, 2),     # decode rows, the projections' reduction split
    (256, 2, 70, 512, 8, 4),    # Gemma-2's head dim, block rows
    (40, 3, 33, 256, 6, 3),     # a head dim padded to 64 in the cache
])
def test_qkv_append_other_head_dims(gpu, hd, n_seq, n_tok, dim, n_head, n_kv):
    """main_qkv at head dims other than 64 and 128 (the reference takes any multiple of 8,
    kv_cache.rs:150-156): projection kernel for q, K and V, then the append -- projections
    within tolerance, codes bit-exact with the oracle's append of the returned K and V, and the
    same q and cache bits when K and V are staged in the workspace instead."""
    say(f"qkv other hd={hd} n_seq={n_seq} n_tok={n_tok} dim={dim}")
    rng = np.random.default_rng(hd + n_tok)
    max_seq = 128 + n_tok + 16
    p = Pair(n_seq, n_kv, hd, max_seq, 1e6)
    lens = rng.integers(0, 100, size=n_seq).astype(np.int32)
    p.set_lens(lens)
    x, (wq, wk, wv), q, lens_before = run_case(p, rng, n_tok, dim, n_head)
    g2 = KVCache.new_int4(1, n_kv, hd, max_seq, n_seq)
    for s, l in enumerate(lens_before):
        g2.set_seq_len(int(l), seq=s)
    q2 = g2.qkv_append(0, dev(x), dev(wq), dev(wk), dev(wv), p.rope).cpu().numpy()
    assert np.array_equal(q2.view(np.uint32), q.view(np.uint32))
    torch.cuda.synchronize()
    for s in range(n_seq):
        a = [t.cpu() for t in p.gpu.export(0, s, int(lens_before[s]), n_tok)]
        b = [t.cpu() for t in g2.export(0, s, int(lens_before[s]), n_tok)]
        for u, w in zip(a, b):
            assert torch.equal(u.view(torch.uint8), w.view(torch.uint8))
