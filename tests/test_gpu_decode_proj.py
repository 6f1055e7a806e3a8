"""GPU parity of ts_attn_decode_append_proj: one decode token per sequence through the append,
the split-K attention and the output projection with the residual add, the split-K combine
merged inside the projection.  The attention output within |err| <= 2e-3 + 1e-3*|ref| of the
oracle's attention (main_attn_out_int4 semantics), the stashed dot and act within the same
bound of the oracle's projection (or_attn_proj) of the GPU's attention output, and the
appended rows bit-exact.  Ragged lengths give some sequences many splits and some one (whose
output the decode writes directly)."""
import numpy as np
import pytest
import torch

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say
from oracle import oracle

pytestmark = pytest.mark.gpu


def fill(p: Pair, rng, lens, step=512):
    done = np.zeros(p.n_seq, np.int64)
    while (done < lens).any():
        m = step
        k = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd))
        v = synth.normal(rng, (p.n_seq, m, p.n_kv, p.hd))
        p.append(k, v)
        p.advance(m)
        done += m
    p.set_lens(lens)


@pytest.mark.parametrize("n_seq,n_kv,hd,n_head,lens,dim", [
    (4, 8, 128, 32, [3000, 100, 1200, 2500], 4096),   # many splits, one sequence with one split
    (3, 2, 64, 16, [1800, 700, 64], 2048),            # head_dim 64, G = 8
    (2, 4, 128, 20, [900, 1500], 1000),               # dim not a multiple of the column tile
])
def test_decode_append_proj(gpu, n_seq, n_kv, hd, n_head, lens, dim):
    say(f"decode_append_proj S={n_seq} kv={n_kv} hd={hd} heads={n_head} lens={lens} dim={dim}")
    rng = np.random.default_rng(sum(lens) + dim)
    lens = np.asarray(lens, np.int64)
    p = Pair(n_seq, n_kv, hd, int(lens.max()) + 600, 500000.0)
    fill(p, rng, lens)
    K = n_head * hd
    wo = (rng.standard_normal((dim, K)) * 0.02).astype(np.float16)
    act0 = rng.standard_normal((n_seq, dim)).astype(np.float32) * 4
    wo_d = dev(wo)
    for step in range(2):
        k = synth.normal(rng, (n_seq, 1, n_kv, hd))
        v = synth.normal(rng, (n_seq, 1, n_kv, hd))
        q = synth.normal(rng, (n_seq, n_head, hd))
        act_d = dev(act0)
        stash_d = torch.zeros((n_seq, dim), dtype=torch.float32, device="cuda")
        out = p.gpu.attn_decode_append_proj(0, dev(k), dev(v), dev(q), p.rope, wo_d, act_d, stash=stash_d)
        torch.cuda.synchronize()
        p.ora.append(k, v)
        ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
        g_out = out.cpu().numpy()
        assert_close(g_out, ref, f"step {step} attention output")
        ref_act, ref_dot = oracle.attn_proj(g_out.reshape(n_seq, K), wo.view(np.uint16), act0)
        assert_close(stash_d.cpu().numpy(), ref_dot, f"step {step} projection")
        assert_close(act_d.cpu().numpy(), ref_act, f"step {step} residual + projection")
        p.advance(1)
    p.check_codes()
