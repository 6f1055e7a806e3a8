"""GPU parity of the attention output projection with the residual add (main_attn_proj,
sh_layer_v1.wgsl:763-821, F16 weights): the stashed dot within |err| <= 2e-3 + 1e-3*|ref| of
the oracle's f32 dot, and act updated to act + dot within the same bound, for decode batches
(the split reduction), prefill chunks (64-row tiles with ragged last tiles), column counts that
are not a multiple of the 256-column tile, and a reduction length that cannot be split."""
import numpy as np
import pytest
import torch

from airframe_amd import TsError
from airframe_amd.kv_cache import attn_out_proj
from tests.gpu_util import assert_close, dev, say
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_tok,attn_dim,dim", [
    (32, 4096, 4096),   # Qwen3-8B / Llama-3-8B shape, decode batch 32: split reduction
    (1, 3072, 3072),    # Llama-3.2-3B, one token
    (300, 2048, 2560),  # prefill chunk: 64-row tiles, the last one ragged
    (5, 320, 200),      # attn_dim not a multiple of 256 (no split), dim not of 256
])
def test_attn_out_proj(gpu, n_tok, attn_dim, dim):
    say(f"attn_out_proj n_tok={n_tok} attn_dim={attn_dim} dim={dim}")
    rng = np.random.default_rng(n_tok + attn_dim + dim)
    a = rng.standard_normal((n_tok, attn_dim)).astype(np.float32)
    wo = (rng.standard_normal((dim, attn_dim)) * 0.02).astype(np.float16)
    act = rng.standard_normal((n_tok, dim)).astype(np.float32) * 4
    act_d, stash_d = dev(act), torch.zeros((n_tok, dim), dtype=torch.float32, device="cuda")
    attn_out_proj(dev(a), dev(wo), act_d, stash=stash_d)
    torch.cuda.synchronize()
    ref_act, ref_dot = oracle.attn_proj(a, wo.view(np.uint16), act)
    assert_close(stash_d.cpu().numpy(), ref_dot, "projection")
    assert_close(act_d.cpu().numpy(), ref_act, "residual + projection")
    # without a stash: the same act bits
    act2 = dev(act)
    attn_out_proj(dev(a), dev(wo), act2)
    assert torch.equal(act2, act_d)


def test_attn_out_proj_errors(gpu):
    say("attn_out_proj errors")
    a = dev(np.zeros((2, 100), np.float32))
    with pytest.raises(TsError) as e:
        attn_out_proj(a, dev(np.zeros((64, 100), np.float16)), dev(np.zeros((2, 64), np.float32)))
    assert e.value.code == -1
    a = dev(np.zeros((2, 4096), np.float32))
    with pytest.raises(TsError) as e:
        attn_out_proj(a, dev(np.zeros((64, 4096), np.float16)), dev(np.zeros((2, 64), np.float32)),
                      workspace=torch.empty(16, dtype=torch.uint8, device="cuda"))
    assert e.value.code == -6
