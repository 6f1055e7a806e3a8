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


def replay_check(p: Pair, rng, n_head, n_replays, advance=False):
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
        if advance:  # the step's last layer: the lengths advance inside the decode launch
            p.gpu.attn_decode_append(0, k_in, v_in, q_in, p.rope, out=out, workspace=ws, advance=True)
        else:
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


def test_graph_replays_advance_in_combine(gpu):
    """ts_attn_decode_append_advance captured once: the combine kernel advances the lengths (the
    last of its workgroups to arrive), so no length-update launch; five replays across split
    and window boundaries, each against the oracle at the advanced lengths."""
    say("graph replays advance in combine")
    rng = np.random.default_rng(320)
    lens = [2047, 1023, 4000, 63, 1500, 255]
    p = Pair(len(lens), 2, 128, 4100, 1e6)
    fill(p, rng, max(lens))
    p.set_lens(lens)
    replay_check(p, rng, 8, 5, advance=True)


def test_graph_replays_advance_without_split(gpu):
    """The same for a plan without a split (256 streams, one workgroup each): the length update
    follows the decode launch."""
    say("graph replays advance, no split")
    rng = np.random.default_rng(321)
    lens = [int(x) for x in rng.integers(1000, 1100, size=32)]
    p = Pair(len(lens), 8, 128, 1110, 1e6)
    fill(p, rng, max(lens), step=1024)
    p.set_lens(lens)
    replay_check(p, rng, 32, 3, advance=True)


@pytest.mark.parametrize("hd,n_kv,n_head,len0", [(64, 8, 32, 508), (128, 4, 12, 509)])
def test_graph_replays_wide_plan(gpu, hd, n_kv, n_head, len0):
    """Batch 1 with 8 windows before the new token: the captured plan is one 8-wave workgroup
    per stream, no split, the lengths advanced inside the decode kernel.  Replays run the
    length past 512, where one wave streams a second window the captured plan did not count
    on."""
    say(f"graph replays wide plan hd={hd} len0={len0}")
    rng = np.random.default_rng(330 + hd)
    p = Pair(1, n_kv, hd, 530, 1e6)
    fill(p, rng, len0)
    p.set_lens([len0])
    replay_check(p, rng, n_head, 7, advance=True)


def test_advance_matches_decode_then_increment(gpu):
    """Eager: decode_append(advance=True) gives bit-identical outputs and cache contents to
    decode_append followed by increment(1), and the same lengths, for a split plan (batch 1)."""
    say("advance vs increment")
    rng = np.random.default_rng(322)
    a = Pair(1, 8, 128, 700, 500000.0)
    b = Pair(1, 8, 128, 700, 500000.0)
    for t0 in range(0, 600, 200):
        k = synth.normal(rng, (1, 200, 8, 128))
        v = synth.normal(rng, (1, 200, 8, 128))
        for c in (a, b):
            c.append(k, v)
            c.advance(200)
    for step in range(3):
        k = dev(synth.normal(rng, (1, 1, 8, 128)))
        v = dev(synth.normal(rng, (1, 1, 8, 128)))
        q = dev(synth.normal(rng, (1, 32, 128)))
        oa = a.gpu.attn_decode_append(0, k, v, q, a.rope, advance=True)
        ob = b.gpu.attn_decode_append(0, k, v, q, b.rope)
        b.gpu.increment(1)
        torch.cuda.synchronize()
        assert torch.equal(oa, ob), f"step {step}: outputs differ"
        assert a.gpu.get_seq_len(0) == b.gpu.get_seq_len(0) == 600 + step + 1
    for x, y in zip(a.gpu.export(0, 0, 0, 603), b.gpu.export(0, 0, 0, 603)):
        assert torch.equal(x, y)


@pytest.mark.parametrize("n_head", [32, 64])
def test_graph_replays_g4_kernel(gpu, n_head):
    """Batch 8 of 4K-8K contexts, 8 kv heads with 4 or 8 query heads each (the integer kernel,
    splits of 1024 and more), with two sequences one short of a multiple of 1024; four
    replays."""
    say(f"graph replays integer kernel, {n_head} q heads")
    rng = np.random.default_rng(310)
    lens = [8191, 8000, 6143, 7000, 5000, 8100, 4095, 6500]
    p = Pair(len(lens), 8, 128, 8300, 1e6)
    fill(p, rng, max(lens), step=1024)
    p.set_lens(lens)
    replay_check(p, rng, n_head, 4)


def test_graph_replays_noalloc_bit_identical(gpu):
    """ts_attn_decode_append_noalloc (partials in the library's scratch array) captured with the
    increment and replayed: on a twin cache driven eagerly through the workspace entry point,
    every replay's output and appended rows are bit-identical."""
    import ctypes

    from airframe_amd import _lib
    from airframe_amd.kv_cache import KVCache, RopeTable, _stream

    say("graph replays noalloc")
    n_seq, n_kv, hd, n_head = 4, 8, 128, 32
    max_seq = 8448
    rope = RopeTable(max_seq, hd, 1e6)
    rng = np.random.default_rng(320)
    a = KVCache.new_int4(1, n_kv, hd, max_seq, n_seq)
    b = KVCache.new_int4(1, n_kv, hd, max_seq, n_seq)
    for t0 in range(0, 8200, 2050):
        k = dev(synth.normal(rng, (n_seq, 2050, n_kv, hd)))
        v = dev(synth.normal(rng, (n_seq, 2050, n_kv, hd)))
        for c in (a, b):
            c.append_quant(0, k, v, rope)
            c.increment(2050)
    lens = [8191, 5119, 7000, 4095]
    for c in (a, b):
        for s, l in enumerate(lens):
            c.set_seq_len(l, seq=s)
    k_in = torch.zeros((n_seq, 1, n_kv, hd), device="cuda")
    v_in = torch.zeros((n_seq, 1, n_kv, hd), device="cuda")
    q_in = torch.zeros((n_seq, n_head, hd), device="cuda")
    out = torch.empty((n_seq, n_head, hd), device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=cap):
        rc = _lib.load().ts_attn_decode_append_noalloc(
            b.handle, 0, ctypes.c_void_p(k_in.data_ptr()), ctypes.c_void_p(v_in.data_ptr()),
            ctypes.c_void_p(q_in.data_ptr()), n_head, rope.handle, ctypes.c_float(0.0),
            ctypes.c_void_p(out.data_ptr()), _stream())
        b.increment(1)
    assert rc == 0, _lib.load().ts_status_string(rc)
    torch.cuda.synchronize()
    for r in range(4):
        k = dev(synth.normal(rng, (n_seq, 1, n_kv, hd)))
        v = dev(synth.normal(rng, (n_seq, 1, n_kv, hd)))
        q = dev(synth.normal(rng, (n_seq, n_head, hd)))
        k_in.copy_(k)
        v_in.copy_(v)
        q_in.copy_(q)
        graph.replay()
        ref = a.attn_decode_append(0, k, v, q, rope)
        a.increment(1)
        torch.cuda.synchronize()
        ro, oo = ref.cpu().numpy(), out.cpu().numpy()
        assert np.array_equal(ro.view(np.uint32), oo.view(np.uint32)), f"replay {r}: max diff {np.abs(ro - oo).max()}"
        for s, l in enumerate(lens):
            for x, y in zip(a.export(0, s, l + r, 1), b.export(0, s, l + r, 1)):
                assert torch.equal(x, y), f"replay {r} sequence {s}: appended row differs"
    del graph


def test_graph_replays_prefill_chunks(gpu):
    """Append + chunked prefill + increment of a 96-token chunk captured once and replayed for
    three consecutive chunks of a ragged batch: every replay against the oracle, codes
    bit-exact after."""
    say("graph replays prefill")
    rng = np.random.default_rng(330)
    n_kv, hd, n_head, C = 4, 128, 16, 96
    lens = [0, 130, 517]
    p = Pair(len(lens), n_kv, hd, 1000, 1e6)
    fill(p, rng, max(lens))
    p.set_lens(lens)
    B = len(lens)
    k_in = torch.zeros((B, C, n_kv, hd), device="cuda")
    v_in = torch.zeros((B, C, n_kv, hd), device="cuda")
    q_in = torch.zeros((B, C, n_head, hd), device="cuda")
    out = torch.empty((B, C, n_head, hd), device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=cap):
        p.gpu.append_quant(0, k_in, v_in, p.rope)
        p.gpu.attn_prefill(0, q_in, p.rope, out=out)
        p.gpu.increment(C)
    torch.cuda.synchronize()
    for r in range(3):
        k = synth.normal(rng, (B, C, n_kv, hd))
        v = synth.normal(rng, (B, C, n_kv, hd))
        q = synth.normal(rng, (B, C, n_head, hd))
        k_in.copy_(dev(k))
        v_in.copy_(dev(v))
        q_in.copy_(dev(q))
        graph.replay()
        torch.cuda.synchronize()
        p.ora.append(k, v)
        ref = p.ora.attend(q, C, threads=8)
        p.ora.advance(C)
        assert_close(out.cpu().numpy(), ref, f"prefill replay {r} at {p.ora.lens.tolist()}")
    del graph
    p.set_lens(p.ora.lens.copy())
    p.check_codes()


def test_graph_replays_qkv_append_other_head_dim(gpu):
    """ts_qkv_append at head_dim 96 (projection kernels onto zeroed outputs -- a fill kernel,
    no memset -- then the append, K and V staged in the workspace) and the increment, captured
    once and replayed for three tokens: q and the appended cache bits of every replay identical
    to the same call made eagerly on a second cache, q within tolerance of the oracle."""
    from airframe_amd.kv_cache import KVCache
    from oracle import oracle
    say("graph replays qkv_append hd 96")
    rng = np.random.default_rng(96)
    B, n_kv, hd, n_head, dim = 3, 2, 96, 8, 512
    lens = [0, 40, 77]
    p = Pair(B, n_kv, hd, 200, 1e6)
    p.set_lens(lens)
    g2 = KVCache.new_int4(1, n_kv, hd, 200, B)
    for s, l in enumerate(lens):
        g2.set_seq_len(l, seq=s)
    wq = (rng.standard_normal((n_head * hd, dim)) * 0.02).astype(np.float16)
    wk = (rng.standard_normal((n_kv * hd, dim)) * 0.02).astype(np.float16)
    wv = (rng.standard_normal((n_kv * hd, dim)) * 0.02).astype(np.float16)
    wq_d, wk_d, wv_d = dev(wq), dev(wk), dev(wv)
    x_in = torch.zeros((B, 1, dim), device="cuda")
    q_out = torch.empty((B, 1, n_head, hd), device="cuda")
    ws = p.gpu.qkv_workspace(dim, 1, n_head)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=cap):
        p.gpu.qkv_append(0, x_in, wq_d, wk_d, wv_d, p.rope, q_out=q_out, workspace=ws)
        p.gpu.increment(1)
    torch.cuda.synchronize()
    for r in range(3):
        x = rng.standard_normal((B, 1, dim)).astype(np.float32)
        x_in.copy_(dev(x))
        graph.replay()
        torch.cuda.synchronize()
        q2 = g2.qkv_append(0, dev(x), wq_d, wk_d, wv_d, p.rope).cpu()
        g2.increment(1)
        torch.cuda.synchronize()
        assert torch.equal(q_out.cpu().view(torch.int32), q2.view(torch.int32)), f"replay {r}: q"
        assert_close(q_out.cpu().numpy().reshape(B, -1), oracle.project(x.reshape(B, dim), wq.view(np.uint16)),
                     f"replay {r}: q against the oracle")
        for s in range(B):
            a = [t.cpu() for t in p.gpu.export(0, s, lens[s] + r, 1)]
            b = [t.cpu() for t in g2.export(0, s, lens[s] + r, 1)]
            for u, w in zip(a, b):
                assert torch.equal(u.view(torch.uint8), w.view(torch.uint8)), f"replay {r}: codes of seq {s}"
    del graph


def test_eager_after_replays_reads_device_lengths(gpu):
    """Batch 1: eager decode calls take the host's length as a launch argument (as the
    reference passes its uniforms).  Once a call that advances the lengths has been captured,
    replays move the device length past the host's; the eager calls after them must read the
    device length (no host resynchronisation in between) and still match the oracle."""
    say("eager decode after replays that advanced the device length")
    rng = np.random.default_rng(330)
    n_head = 8
    p = Pair(1, 2, 128, 3000, 1e6)
    fill(p, rng, 1500)

    def eager_step(advance):
        k = synth.normal(rng, (1, 1, 2, 128))
        v = synth.normal(rng, (1, 1, 2, 128))
        q = synth.normal(rng, (1, n_head, 128))
        out = p.gpu.attn_decode_append(0, dev(k), dev(v), dev(q), p.rope, advance=advance).cpu().numpy()
        p.ora.append(k, v)
        ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
        p.ora.advance(1)
        if not advance:
            p.gpu.increment(1)
        return out, ref

    for t in range(2):  # eager: the host length as the launch argument
        out, ref = eager_step(advance=t == 1)
        assert_close(out, ref, f"eager step {t}")
    k_in = torch.zeros((1, 1, 2, 128), device="cuda")
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros((1, n_head, 128), device="cuda")
    out = torch.empty((1, n_head, 128), device="cuda")
    ws = p.gpu.workspace(n_head)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=cap):
        p.gpu.attn_decode_append(0, k_in, v_in, q_in, p.rope, out=out, workspace=ws, advance=True)
    torch.cuda.synchronize()
    for r in range(3):
        k = synth.normal(rng, (1, 1, 2, 128))
        v = synth.normal(rng, (1, 1, 2, 128))
        q = synth.normal(rng, (1, n_head, 128))
        k_in.copy_(dev(k))
        v_in.copy_(dev(v))
        q_in.copy_(dev(q))
        graph.replay()
        torch.cuda.synchronize()
        p.ora.append(k, v)
        ref = p.ora.attend(q[:, None], 1, threads=8)[:, 0]
        p.ora.advance(1)
        assert_close(out.cpu().numpy(), ref, f"replay {r}")
    del graph
    # the host length advanced once (at capture), the device's three times: 2 ahead
    assert p.gpu.get_seq_len(0) == int(p.ora.lens[0]) - 2
    out, ref = eager_step(advance=False)
    assert_close(out, ref, "eager step after the replays, at the device length")
    p.check_codes()
