"""Seeded random shapes through the projections: the QKV projection with the INT4 append as its
epilogue and the output projection with the residual add, for every weight form the path takes
(f16 rows, two f16 planes converted from a GGUF blob, and the GGUF blocks read in the loop),
with ragged cache lengths, decode and block rows, split and unsplit reductions and head dims
outside 64/128.  Projections within 2e-3 + 1e-3 |ref| of the oracle's f32 dot over the exact
weights, appended codes bit-exact."""
import numpy as np
import pytest
import torch

from airframe_amd import weights
from airframe_amd.kv_cache import attn_out_proj, attn_out_proj_gguf
from oracle import oracle
from tests.gpu_util import Pair, assert_close, dev, say
from tests.test_gpu_weights import random_blob

pytestmark = pytest.mark.gpu

IN_LOOP = (weights.Q4_K, weights.Q5_K, weights.Q8_0, weights.Q4_0, weights.Q5_0)
CONVERTED = (weights.F32, weights.Q6_K, weights.Q8_0, weights.Q4_K)


def draw_weights(rng, form, fmt, rows, dim):
    """(device weights, exact f32 weights [rows][dim]) of one matrix in the given form."""
    if form == "f16":
        w = (rng.standard_normal((rows, dim)) * 0.02).astype(np.float16)
        return dev(w), w.astype(np.float32)
    blob = random_blob(rng, fmt, rows, dim)
    wf = oracle.dequant(fmt, blob, rows * dim).reshape(rows, dim)
    if form == "planes":
        return weights.to_f16(fmt, dev(blob), rows, dim, planes=2), wf
    return dev(blob), wf


def form_of(rng):
    form = str(rng.choice(["f16", "planes", "blocks"]))
    fmt = int(rng.choice(IN_LOOP if form == "blocks" else CONVERTED)) if form != "f16" else None
    return form, fmt


@pytest.mark.parametrize("seed", range(16))
def test_random_qkv_append(gpu, seed):
    rng = np.random.default_rng(7000 + seed)
    form, fmt = form_of(rng)
    hd = int(rng.choice([40, 64, 96, 128, 128, 256]))
    n_kv = int(rng.choice([1, 2, 4]))
    n_head = n_kv * int(rng.integers(1, 7))
    n_seq = int(rng.integers(1, 41))
    n_tok = 1 if rng.integers(0, 2) == 0 else int(rng.integers(2, 81))
    if n_tok > 1:
        n_seq = min(n_seq, 4)
    dim = 256 * int(rng.integers(1, 13)) if form == "blocks" else 64 * int(rng.integers(1, 49))
    if form == "planes" and fmt != weights.F32:
        dim = -(-dim // 256) * 256  # whole blocks per row
    say(f"random qkv seed={seed} form={form} fmt={fmt} hd={hd} n_kv={n_kv} n_head={n_head} "
        f"n_seq={n_seq} n_tok={n_tok} dim={dim}")
    fill = int(rng.integers(0, 200))
    p = Pair(n_seq, n_kv, hd, fill + n_tok + 8, 500000.0)
    if fill:
        p.append(rng.standard_normal((n_seq, fill, n_kv, hd)).astype(np.float32),
                 rng.standard_normal((n_seq, fill, n_kv, hd)).astype(np.float32))
        p.set_lens([int(x) for x in rng.integers(0, fill + 1, size=n_seq)])
    rows = (n_head * hd, n_kv * hd, n_kv * hd)
    ws = [draw_weights(rng, form, fmt, r, dim) for r in rows]
    x = rng.standard_normal((n_seq, n_tok, dim)).astype(np.float32)
    k_out = torch.empty((n_seq, n_tok, n_kv, hd), dtype=torch.float32, device="cuda")
    v_out = torch.empty_like(k_out)
    if form == "blocks":
        q = p.gpu.qkv_append_gguf(0, dev(x), fmt, ws[0][0], ws[1][0], ws[2][0], p.rope, kv_out=(k_out, v_out))
    else:
        q = p.gpu.qkv_append(0, dev(x), ws[0][0], ws[1][0], ws[2][0], p.rope, kv_out=(k_out, v_out),
                             planes=2 if form == "planes" else 1)
    torch.cuda.synchronize()
    q, k_out, v_out = q.cpu().numpy(), k_out.cpu().numpy(), v_out.cpu().numpy()
    xf = x.reshape(-1, dim)
    for name, got, (_, wf) in (("q", q, ws[0]), ("k", k_out, ws[1]), ("v", v_out, ws[2])):
        assert_close(got.reshape(n_seq * n_tok, -1), oracle.project_f32(xf, wf), f"{name} projection")
    p.ora.append(k_out, v_out)
    p.advance(n_tok)
    p.check_codes()


@pytest.mark.parametrize("seed", range(12))
def test_random_attn_out_proj(gpu, seed):
    rng = np.random.default_rng(8000 + seed)
    form, fmt = form_of(rng)
    n_tok = 1 if rng.integers(0, 2) == 0 else int(rng.integers(2, 300))
    attn_dim = 256 * int(rng.integers(1, 13)) if form != "f16" else 64 * int(rng.integers(1, 49))
    dim = int(rng.integers(1, 40)) * 64
    say(f"random attn_out_proj seed={seed} form={form} fmt={fmt} n_tok={n_tok} attn_dim={attn_dim} dim={dim}")
    w, wf = draw_weights(rng, form, fmt, dim, attn_dim)
    a = rng.standard_normal((n_tok, attn_dim)).astype(np.float32)
    act = rng.standard_normal((n_tok, dim)).astype(np.float32) * 4
    act_d = dev(act)
    stash = torch.zeros((n_tok, dim), dtype=torch.float32, device="cuda")
    if form == "blocks":
        attn_out_proj_gguf(dev(a), fmt, w, dim, act_d, stash=stash)
    else:
        attn_out_proj(dev(a), w, act_d, stash=stash, planes=2 if form == "planes" else 1)
    torch.cuda.synchronize()
    dot = oracle.project_f32(a, wf)
    assert_close(stash.cpu().numpy(), dot, "projection")
    assert_close(act_d.cpu().numpy(), act + dot, "residual + projection")
