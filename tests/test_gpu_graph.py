"""The fused decode (ts_attn_decode_append) and the length increment captured once in a HIP
graph and replayed while the device lengths grow.  The split plan is fixed at capture; the
kernels read the lengths on the device and the last split of a sequence runs to its end, so
every replay must still match the oracle (|err| <= 2e-3 + 1e-3*|ref|) and leave bit-exact codes,
also when a sequence crosses a split boundary between replays.  Eager work and a
synchronization separate the replays."""
import numpy as np
import pytest
import torch

from airframe_amd import synth
from tests.gpu_util import Pair, assert_close, dev, say
from tests.test_gpu_decode_append import fill

pytestmark = pytest.mark.gpu


def replay_check(p: Pair, rng, n_head, n_replays):
    B, n_kv, hd = p.n_seq, p.n_kv, p.hd
    k_in = torch.zeros((B, 1, n_kv, hd), device="cuda")
    v_in = torch.zeros((B, 1, n_kv, hd), device="cuda")
    q_in = torch.zeros((B, n_head, hd), device="cuda")
    out = torch.empty((B, n_head, hd), device="cuda")
    ws = p.gpu.workspace(n_head)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=cap):
        p.gpu.attn_decode_append(0, k_in, v_in, q_in, p.rope, out=out, workspace=ws)
        p.gpu.increment(1)
    torch.cuda.synchronize()
    for r in range(n_replays):
        k = synth.normal(rng, (B, 1, n_kv, hd))
        v = synth.normal(rng, (B, 1, n_kv, hd))
        q = synth.normal(rng, (B, n_head, hd))
        k_in.copy_(dev(k))
        v_in.copy_(dev(v))
        q_in.copy_(dev(q))
        graph.replay()
        torch.cuda.synchronize()
        p.ora.append(k, v)
        ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
        p.ora.advance(1)
        assert_close(out.cpu().numpy(), ref, f"replay {r} at {p.ora.lens.tolist()}")
    del graph
    # the host mirror advanced once, at capture; the device once per replay
    p.set_lens(p.ora.lens.copy())
    p.check_codes()


@pytest.mark.parametrize("n_head", [8, 16])
def test_graph_replays_ragged_split_edges(gpu, n_head):
    """Short ragged batch (16x16 kernel, splits of 256): lengths one short of split and window
    boundaries, five replays."""
    say(f"graph replays ragged n_head={n_head}")
    rng = np.random.default_rng(300 + n_head)
    lens = [2047, 1023, 4000, 63, 1500, 255]
    p = Pair(len(lens), 2, 128, 4100, 1e6)
    fill(p, rng, max(lens))
    p.set_lens(lens)
    replay_check(p, rng, n_head, 5)


def test_graph_replays_g4_kernel(gpu):
    """Batch 8 of 4K-8K contexts, 32/8 heads (the G <= 4 kernel, splits of 1024 and more), with
    two sequences one short of a multiple of 1024; four replays."""
    say("graph replays G<=4 kernel")
    rng = np.random.default_rng(310)
    lens = [8191, 8000, 6143, 7000, 5000, 8100, 4095, 6500]
    p = Pair(len(lens), 8, 128, 8300, 1e6)
    fill(p, rng, max(lens), step=1024)
    p.set_lens(lens)
    replay_check(p, rng, 32, 4)
