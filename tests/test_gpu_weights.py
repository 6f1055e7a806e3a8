"""GPU conversion of GGUF projection weights (ts_weights_to_f16) against the oracle's
dequantizers (src/core/dequant/, pinned in test_oracle_weights.py): every element bit-exact
with the oracle's f32 value rounded to f16 (nearest even).  Then the projections fed with
converted weights against the reference's f32-weight dot (main_qkv's block branch), within
|err| <= 2e-3 + 1e-3*|ref| -- the f16 rounding of the weights included."""
import numpy as np
import pytest
import torch

from airframe_amd import weights
from airframe_amd.kv_cache import attn_out_proj, attn_out_proj_gguf
from oracle import oracle
from tests.gpu_util import Pair, assert_close, dev, say

pytestmark = pytest.mark.gpu

EPB = {weights.F32: 1, weights.F16: 1, weights.Q4_0: 32, weights.Q5_0: 32, weights.Q8_0: 32,
       weights.Q4_K: 256, weights.Q5_K: 256, weights.Q6_K: 256}
BPB = {weights.F32: 4, weights.F16: 2, weights.Q4_0: 18, weights.Q5_0: 22, weights.Q8_0: 34,
       weights.Q4_K: 144, weights.Q5_K: 176, weights.Q6_K: 210}


def f16_bytes(rng, n, lo, hi):
    return np.frombuffer(rng.uniform(lo, hi, n).astype(np.float16).tobytes(), np.uint8).reshape(n, 2)


def random_blob(rng, fmt, n_rows, n_cols, scale=2e-3):
    """Random GGUF bytes of an [n_rows][n_cols] matrix with finite scales of about `scale`."""
    if fmt == weights.F32:
        return (rng.standard_normal(n_rows * n_cols) * 0.02).astype(np.float32).view(np.uint8)
    if fmt == weights.F16:
        return (rng.standard_normal(n_rows * n_cols) * 0.02).astype(np.float16).view(np.uint8)
    nb = n_rows * n_cols // EPB[fmt]
    b = rng.integers(0, 256, (nb, BPB[fmt]), dtype=np.uint8)
    if fmt in (weights.Q4_0, weights.Q5_0, weights.Q8_0):
        b[:, 0:2] = f16_bytes(rng, nb, scale, 4 * scale)
    elif fmt in (weights.Q4_K, weights.Q5_K):
        b[:, 0:2] = f16_bytes(rng, nb, scale / 16, scale / 4)
        b[:, 2:4] = f16_bytes(rng, nb, scale / 16, scale / 4)
    else:
        b[:, 208:210] = f16_bytes(rng, nb, scale / 64, scale / 16)
    return b.reshape(-1)


@pytest.mark.parametrize("fmt", [weights.F32, weights.F16, weights.Q4_0, weights.Q5_0, weights.Q8_0,
                                 weights.Q4_K, weights.Q5_K, weights.Q6_K])
@pytest.mark.parametrize("n_rows,n_cols", [(48, 512), (3, 1280)])
def test_weights_to_f16_bit_exact(gpu, fmt, n_rows, n_cols):
    """One plane: the oracle's value rounded to f16.  Two planes: that (hi), then the rest
    v - hi (exact in f32) rounded to f16 (lo), per row."""
    say(f"weights_to_f16 fmt={fmt} {n_rows}x{n_cols}")
    rng = np.random.default_rng(fmt * 100 + n_rows)
    blob = random_blob(rng, fmt, n_rows, n_cols)
    assert blob.size == weights.src_bytes(fmt, n_rows, n_cols)
    v = oracle.dequant(fmt, blob, n_rows * n_cols).reshape(n_rows, n_cols)
    hi = v.astype(np.float16)
    lo = (v - hi.astype(np.float32)).astype(np.float16)
    out = weights.to_f16(fmt, dev(blob), n_rows, n_cols).cpu().numpy()
    assert np.array_equal(out.view(np.uint16), hi.view(np.uint16))
    out2 = weights.to_f16(fmt, dev(blob), n_rows, n_cols, planes=2).cpu().numpy()
    assert np.array_equal(out2[:, :n_cols].view(np.uint16), hi.view(np.uint16))
    assert np.array_equal(out2[:, n_cols:].view(np.uint16), lo.view(np.uint16))


def test_weights_to_f16_errors(gpu):
    say("weights_to_f16 errors")
    with pytest.raises(Exception):
        weights.src_bytes(weights.Q4_K, 4, 300)  # not a whole number of blocks per row
    with pytest.raises(Exception):
        weights.src_bytes(3, 4, 256)             # Q4_1: not a format of the path
    with pytest.raises(ValueError):
        weights.to_f16(weights.Q8_0, dev(np.zeros(10, np.uint8)), 1, 32)  # too few bytes


@pytest.mark.parametrize("fmt,n_seq,n_tok,dim", [
    (weights.Q4_K, 8, 1, 4096),    # decode rows: the reduction split over workgroups
    (weights.Q5_K, 3, 70, 1024),   # block rows: one workgroup per tile over all of dim
    (weights.F32, 2, 33, 512),     # the F32 branch
    (weights.Q8_0, 40, 1, 320),    # decode rows in 64-row tiles, dim not a multiple of 256
])
def test_qkv_append_with_block_weights(gpu, fmt, n_seq, n_tok, dim):
    """main_qkv with F32 / block weights (sh_layer_v1_int4.wgsl:502-520): two-plane f16 weights
    through ts_qkv_append_x2 against the dot over the exact dequantized f32 weights, and the
    appended codes bit-exact with the quantizer applied to those projections."""
    say(f"qkv_append_x2 fmt={fmt} n_seq={n_seq} n_tok={n_tok} dim={dim}")
    rng = np.random.default_rng(fmt + dim)
    n_head, n_kv, hd = 8, 2, 128
    p = Pair(n_seq, n_kv, hd, 128, 500000.0)
    rows = (n_head * hd, n_kv * hd, n_kv * hd)
    blobs = [random_blob(rng, fmt, r, dim) for r in rows]
    w2 = [weights.to_f16(fmt, dev(b), r, dim, planes=2) for b, r in zip(blobs, rows)]
    wf = [oracle.dequant(fmt, b, r * dim).reshape(r, dim) for b, r in zip(blobs, rows)]
    x = rng.standard_normal((n_seq, n_tok, dim)).astype(np.float32)
    k_out = torch.empty((n_seq, n_tok, n_kv, hd), dtype=torch.float32, device="cuda")
    v_out = torch.empty_like(k_out)
    q = p.gpu.qkv_append(0, dev(x), w2[0], w2[1], w2[2], p.rope, kv_out=(k_out, v_out), planes=2)
    torch.cuda.synchronize()
    q, k_out, v_out = q.cpu().numpy(), k_out.cpu().numpy(), v_out.cpu().numpy()
    xf = x.reshape(-1, dim)
    assert_close(q.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[0]), "q (block weights)")
    assert_close(k_out.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[1]), "k (block weights)")
    assert_close(v_out.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[2]), "v (block weights)")
    p.ora.append(k_out, v_out)
    p.advance(n_tok)
    p.check_codes()


@pytest.mark.parametrize("fmt,n_tok,attn_dim,dim", [
    (weights.Q6_K, 5, 2048, 2048),   # decode: the reduction split
    (weights.Q8_0, 130, 1024, 768),  # prefill: 64-row tiles over all of attn_dim
    (weights.Q4_0, 3, 320, 200),     # attn_dim not a multiple of 256
])
def test_attn_out_proj_with_block_weights(gpu, fmt, n_tok, attn_dim, dim):
    """main_attn_proj with block-format weights (sh_layer_v1.wgsl:782-790) through
    ts_attn_out_proj_x2."""
    say(f"attn_out_proj_x2 fmt={fmt} n_tok={n_tok} attn_dim={attn_dim} dim={dim}")
    rng = np.random.default_rng(fmt + n_tok)
    blob = random_blob(rng, fmt, dim, attn_dim)
    w2 = weights.to_f16(fmt, dev(blob), dim, attn_dim, planes=2)
    wf = oracle.dequant(fmt, blob, dim * attn_dim).reshape(dim, attn_dim)
    a = rng.standard_normal((n_tok, attn_dim)).astype(np.float32)
    act = rng.standard_normal((n_tok, dim)).astype(np.float32) * 4
    act_d = dev(act)
    stash = torch.zeros((n_tok, dim), dtype=torch.float32, device="cuda")
    attn_out_proj(dev(a), w2, act_d, stash=stash, planes=2)
    torch.cuda.synchronize()
    dot = oracle.project_f32(a, wf)
    assert_close(stash.cpu().numpy(), dot, "projection (block weights)")
    assert_close(act_d.cpu().numpy(), act + dot, "residual + projection (block weights)")


@pytest.mark.parametrize("fmt,n_seq,n_tok,dim,hd", [
    (weights.Q4_K, 8, 1, 4096, 128),   # decode rows: the reduction split over workgroups
    (weights.Q5_K, 32, 1, 2048, 128),  # a full 32-row decode tile
    (weights.Q4_K, 3, 70, 1024, 128),  # block rows (prefill chunk)
    (weights.Q5_K, 2, 1, 512, 64),     # head dim 64
    (weights.Q4_K, 4, 1, 768, 96),     # head dim 96: three projections, then the append
    (weights.Q8_0, 8, 1, 4096, 128),   # 32-element blocks: decode rows, split reduction
    (weights.Q4_0, 32, 1, 2048, 128),  # a full 32-row decode tile
    (weights.Q8_0, 3, 70, 1024, 128),  # block rows
    (weights.Q4_0, 2, 1, 512, 64),     # head dim 64
    (weights.Q8_0, 4, 1, 768, 96),     # head dim 96
    (weights.Q5_0, 8, 1, 2048, 128),
    (weights.Q5_0, 3, 70, 1024, 128),
    (weights.Q5_0, 4, 1, 768, 96),
])
def test_qkv_append_gguf_blocks_in_loop(gpu, fmt, n_seq, n_tok, dim, hd):
    """ts_qkv_append_gguf: Q4_K / Q5_K / Q8_0 / Q4_0 / Q5_0 blocks read inside the projection loop, against the dot
    over the oracle's exact dequantized f32 weights (q4_k.rs / q5_k.rs, pinned in
    test_oracle_weights.py), and the appended codes bit-exact with the quantizer applied to
    those projections."""
    say(f"qkv_append_gguf fmt={fmt} n_seq={n_seq} n_tok={n_tok} dim={dim} hd={hd}")
    rng = np.random.default_rng(7 * fmt + dim + hd)
    n_head, n_kv = 8, 2
    p = Pair(n_seq, n_kv, hd, 128, 500000.0)
    rows = (n_head * hd, n_kv * hd, n_kv * hd)
    blobs = [random_blob(rng, fmt, r, dim) for r in rows]
    wf = [oracle.dequant(fmt, b, r * dim).reshape(r, dim) for b, r in zip(blobs, rows)]
    x = rng.standard_normal((n_seq, n_tok, dim)).astype(np.float32)
    k_out = torch.empty((n_seq, n_tok, n_kv, hd), dtype=torch.float32, device="cuda")
    v_out = torch.empty_like(k_out)
    q = p.gpu.qkv_append_gguf(0, dev(x), fmt, dev(blobs[0]), dev(blobs[1]), dev(blobs[2]), p.rope,
                              kv_out=(k_out, v_out))
    torch.cuda.synchronize()
    q, k_out, v_out = q.cpu().numpy(), k_out.cpu().numpy(), v_out.cpu().numpy()
    xf = x.reshape(-1, dim)
    assert_close(q.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[0]), "q (blocks in loop)")
    assert_close(k_out.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[1]), "k (blocks in loop)")
    assert_close(v_out.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[2]), "v (blocks in loop)")
    p.ora.append(k_out, v_out)
    p.advance(n_tok)
    p.check_codes()


@pytest.mark.parametrize("fmt,n_tok,attn_dim,dim", [
    (weights.Q4_K, 5, 2048, 2048),    # decode: the reduction split
    (weights.Q5_K, 130, 1024, 768),   # prefill rows, still split
    (weights.Q4_K, 1100, 512, 2304),  # many tiles: one slice over all of attn_dim
    (weights.Q8_0, 5, 2048, 2048),
    (weights.Q4_0, 130, 1024, 768),
    (weights.Q8_0, 1100, 512, 2304),
    (weights.Q4_0, 1, 3072, 3072),    # batch 1 (config 2's attention width)
    (weights.Q5_0, 5, 2048, 2048),
    (weights.Q5_0, 1100, 512, 2304),
])
def test_attn_out_proj_gguf_blocks_in_loop(gpu, fmt, n_tok, attn_dim, dim):
    """ts_attn_out_proj_gguf against the oracle's f32-weight dot and the residual add."""
    say(f"attn_out_proj_gguf fmt={fmt} n_tok={n_tok} attn_dim={attn_dim} dim={dim}")
    rng = np.random.default_rng(fmt + n_tok + 1)
    blob = random_blob(rng, fmt, dim, attn_dim)
    wf = oracle.dequant(fmt, blob, dim * attn_dim).reshape(dim, attn_dim)
    a = rng.standard_normal((n_tok, attn_dim)).astype(np.float32)
    act = rng.standard_normal((n_tok, dim)).astype(np.float32) * 4
    act_d = dev(act)
    stash = torch.zeros((n_tok, dim), dtype=torch.float32, device="cuda")
    attn_out_proj_gguf(dev(a), fmt, dev(blob), dim, act_d, stash=stash)
    torch.cuda.synchronize()
    dot = oracle.project_f32(a, wf)
    assert_close(stash.cpu().numpy(), dot, "projection (blocks in loop)")
    assert_close(act_d.cpu().numpy(), act + dot, "residual + projection (blocks in loop)")


def test_gguf_in_loop_refusals(gpu):
    """Types without an in-loop form (Q6_K) and dims that are not whole 256s are refused."""
    say("gguf in-loop refusals")
    from airframe_amd import TsError
    p = Pair(1, 2, 128, 16, 500000.0)
    x = torch.zeros((1, 1, 512), device="cuda")
    blob6 = dev(np.zeros(weights.src_bytes(weights.Q6_K, 8 * 128, 512), np.uint8))
    kvb = dev(np.zeros(weights.src_bytes(weights.Q6_K, 2 * 128, 512), np.uint8))
    with pytest.raises(TsError):
        p.gpu.qkv_append_gguf(0, x, weights.Q6_K, blob6, kvb, kvb, p.rope)
    with pytest.raises(TsError):  # 320 inputs: not a whole number of 256-element blocks
        attn_out_proj_gguf(torch.zeros((1, 320), device="cuda"), weights.Q4_K,
                           dev(np.zeros(16, np.uint8)), 256, torch.zeros((1, 256), device="cuda"))


@pytest.mark.parametrize("n_tok", [1, 40])
def test_qkv_append_gguf_with_qk_norm(gpu, n_tok):
    """The K-quant projections with Qwen3's QK norm set: the appended K is normalized before its
    rotation (the epilogue shared with the f16 path), codes bit-exact against the oracle's
    append of the kernel's own raw K/V, q returned raw."""
    say(f"qkv_append_gguf with QK norm n_tok={n_tok}")
    rng = np.random.default_rng(940 + n_tok)
    n_seq, n_head, n_kv, hd, dim = 3, 8, 2, 128, 768
    p = Pair(n_seq, n_kv, hd, 128, 1e6)
    wq_n = (rng.standard_normal(hd) * 0.4 + 1.0).astype(np.float32)
    wk_n = (rng.standard_normal(hd) * 0.4 + 1.0).astype(np.float32)
    p.gpu.set_qk_norm(0, dev(wq_n), dev(wk_n), 1e-6)
    p.ora.q_norm, p.ora.k_norm, p.ora.norm_eps = wq_n, wk_n, 1e-6
    rows = (n_head * hd, n_kv * hd, n_kv * hd)
    blobs = [random_blob(rng, weights.Q4_K, r, dim) for r in rows]
    wf = [oracle.dequant(weights.Q4_K, b, r * dim).reshape(r, dim) for b, r in zip(blobs, rows)]
    x = rng.standard_normal((n_seq, n_tok, dim)).astype(np.float32)
    k_out = torch.empty((n_seq, n_tok, n_kv, hd), dtype=torch.float32, device="cuda")
    v_out = torch.empty_like(k_out)
    q = p.gpu.qkv_append_gguf(0, dev(x), weights.Q4_K, dev(blobs[0]), dev(blobs[1]), dev(blobs[2]),
                              p.rope, kv_out=(k_out, v_out))
    torch.cuda.synchronize()
    q, k_out, v_out = q.cpu().numpy(), k_out.cpu().numpy(), v_out.cpu().numpy()
    xf = x.reshape(-1, dim)
    assert_close(q.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[0]), "raw q (QK norm set)")
    assert_close(k_out.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf[1]), "raw k (QK norm set)")
    p.ora.append(k_out, v_out)
    p.advance(n_tok)
    p.check_codes()
