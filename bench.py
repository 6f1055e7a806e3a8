"""Benchmark of the INT4 KV decode path on one MI355X.

Default workload (the headline): Qwen3-8B attention shape, 36 layers,
32 query / 8 kv heads, head_dim 128, batch 32, each sequence with 8192 cached INT4 tokens,
seeded f32 N(0,1) Q/K/V with x8 outlier channels on 2% of dims, RoPE theta 1e6.  A step is one
decode token for all 32 sequences: per layer, RoPE-fused quantize-on-append of the new K/V
and split-K GQA attention over the INT4 cache in one launch (ts_attn_decode_append; with
--separate, ts_append_quant then ts_attn_decode); the lengths advance inside the last layer's
launch (ts_attn_decode_append_advance; --no-fold: a separate ts_kv_increment).
All inputs are generated on the device before timing.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]

Prints one JSON line.  `value` = algorithmic HBM bytes of the whole step / step time (GB/s);
`roofline` = the decode attention kernel (bytes per launch / its average launch time from HIP
events around replays of a graph holding only the layers' decode launches); `cpu_baseline` = the C oracle on a
bounded sample of the same workload (same device-generated inputs copied to the host).
Other configs (--config 1,2,4 decode; 5 chunked prefill) print their own line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

CONFIGS = {
    1: dict(name="llama3.2-1b_b1_ctx512_1layer", layers=1, n_head=32, n_kv=8, hd=64, batch=1,
            ctx=512, theta=500000.0, steps=64, outliers=False, dim=2048),
    2: dict(name="llama3.2-3b_b1_prefill4096_28layers", layers=28, n_head=24, n_kv=8, hd=128,
            batch=1, ctx=4096, theta=500000.0, steps=256, outliers=False, dim=3072),
    3: dict(name="qwen3-8b_b32_ctx8192_36layers", layers=36, n_head=32, n_kv=8, hd=128,
            batch=32, ctx=8192, theta=1000000.0, steps=128, outliers=True, dim=4096),
    4: dict(name="llama3-8b_b8_ctx16k-32k_ragged_32layers", layers=32, n_head=32, n_kv=8, hd=128,
            batch=8, ctx=32768, theta=500000.0, steps=16, outliers=False, ragged=(16384, 32768), dim=4096),
    5: dict(name="qwen3-4b_b4_prefill_4x512_36layers", layers=36, n_head=32, n_kv=8, hd=128,
            batch=4, chunk=512, n_chunks=4, theta=1000000.0, outliers=False, dim=2560),
}


def attn_bytes(batch_ctx, n_kv, n_head, hd, batch):
    """Algorithmic bytes of one decode-attention launch: packed K+V (hd/2 bytes each) and two
    f32 scales for every attended position of every (sequence, kv head), plus q in and o out
    in f32."""
    return sum(batch_ctx) * n_kv * (hd + 8) + 2 * batch * n_head * hd * 4


def append_bytes(batch, n_kv, hd):
    """One appended token per sequence: f32 K and V read, packed rows and scales written."""
    return batch * n_kv * (2 * hd * 4 + hd + 8)


def cpu_threads() -> int:
    """Threads for the OpenMP oracle: the host cores this process may run on (its affinity
    mask), capped by OMP_NUM_THREADS when that is set (the GPU box grants each GPU's jobs a
    share of the host's cores and sets it to that share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_info() -> dict:
    """The host's CPU for the baseline's record: model name, logical CPUs of the host, and the
    CPUs this process may use."""
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = None
    fam = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k in ("cpu family", "model", "stepping", "cpu MHz") and k not in fam:
                    fam[k] = v.strip()
                if line.strip() == "":
                    break
    except OSError:
        pass
    return {"cpu_model": cpu_model(), "cpu_family_model": fam, "host_logical_cpus": os.cpu_count(),
            "affinity_cpus": aff}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(kv, cfg, qs, ks, vs, lens, max_seq, table, layers_mt=2, seqs_st=2, norms=None):
    """Time the C oracle (oracle/ts_oracle.c) on a bounded sample of the same step: append the
    step's token and attend, for every sequence of `layers_mt` layers (OpenMP over
    (sequence, head)) and for `seqs_st` sequences of one layer single-threaded."""
    import torch

    from oracle import oracle
    n_kv, hd, n_head, B = cfg["n_kv"], cfg["hd"], cfg["n_head"], cfg["batch"]
    threads = cpu_threads()
    t_mt = 0.0
    t_st = 0.0
    for layer in range(layers_mt):
        ora = oracle.OracleKV(B, max_seq, n_kv, hd, table)
        if norms is not None:
            ora.q_norm, ora.k_norm = norms[layer]
        for s in range(B):
            kp, vp, kss, vss = kv.export(layer, s, 0, lens[s])
            torch.cuda.synchronize()
            ora.k_packed[s, :lens[s]] = kp.cpu().numpy().view(np.uint32)
            ora.v_packed[s, :lens[s]] = vp.cpu().numpy().view(np.uint32)
            ora.k_scale[s, :lens[s]] = kss.cpu().numpy()
            ora.v_scale[s, :lens[s]] = vss.cpu().numpy()
        ora.lens[:] = np.asarray(lens, np.int32)
        k = ks[layer].cpu().numpy()
        v = vs[layer].cpu().numpy()
        q = qs[layer].cpu().numpy()[:, None]
        t0 = time.perf_counter()
        ora.append(k, v)
        ora.attend(q, 1, threads=threads)
        t_mt += time.perf_counter() - t0
        if layer == 0:
            sub = oracle.OracleKV(seqs_st, max_seq, n_kv, hd, table)
            sub.q_norm, sub.k_norm = ora.q_norm, ora.k_norm
            for name in ("k_packed", "v_packed", "k_scale", "v_scale"):
                getattr(sub, name)[:] = getattr(ora, name)[:seqs_st]
            sub.lens[:] = ora.lens[:seqs_st]
            t0 = time.perf_counter()
            sub.append(k[:seqs_st], v[:seqs_st])
            sub.attend(q[:seqs_st], 1, threads=1)
            t_st = time.perf_counter() - t0
    step_mt = t_mt / layers_mt * cfg["layers"]
    step_st = t_st / seqs_st * B * cfg["layers"]
    return step_mt, threads, step_st


def run_decode(args, cfg):
    import torch

    from airframe_amd import synth
    from airframe_amd.kv_cache import KVCache, RopeTable

    dev = torch.device("cuda:0")
    L, n_head, n_kv, hd, B = cfg["layers"], cfg["n_head"], cfg["n_kv"], cfg["hd"], cfg["batch"]
    steps, warmup = args.steps, args.warmup
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    if "ragged" in cfg:
        rng = np.random.default_rng(args.seed)
        lens0 = [int(x) for x in rng.integers(cfg["ragged"][0], cfg["ragged"][1], size=B)]
    else:
        lens0 = [cfg["ctx"]] * B
    # positions the run appends: the timed steps, or the warmup replays (whole graphs of
    # --steps-per-graph steps each), whichever is more; the device lengths are reset between
    spg = max(1, args.steps_per_graph) if args.graph else 1
    warm_steps = -(-warmup // spg) * spg
    max_seq = max(lens0) + max(steps, warm_steps) + 1
    rope = RopeTable(max_seq, hd, cfg["theta"])
    kv = KVCache.new_int4(L, n_kv, hd, max_seq, B)
    dims = synth.outlier_dims(n_kv, hd, args.seed) if cfg["outliers"] else None
    skv = torch.as_tensor(synth.channel_scale(n_kv, n_kv, hd, dims), device=dev)
    sq = torch.as_tensor(synth.channel_scale(n_head, n_kv, hd, dims), device=dev)

    norms = None
    if args.qk_norm:  # Qwen3's per-head q/K RMSNorm before RoPE, random weights around 1
        norms = []
        for layer in range(L):
            wq = (torch.randn(hd, generator=gen, device=dev) * 0.2 + 1.0).contiguous()
            wk = (torch.randn(hd, generator=gen, device=dev) * 0.2 + 1.0).contiguous()
            kv.set_qk_norm(layer, wq, wk)
            norms.append((wq.cpu().numpy(), wk.cpu().numpy()))

    # Fill every layer's cache to its starting length with the fused append.
    fill = max(lens0)
    chunk = 1024
    for layer in range(L):
        kv.reset()
        for t0 in range(0, fill, chunk):
            m = min(chunk, fill - t0)
            k = torch.randn((B, m, n_kv, hd), generator=gen, device=dev).mul_(skv)
            v = torch.randn((B, m, n_kv, hd), generator=gen, device=dev).mul_(skv)
            kv.append_quant(layer, k, v, rope)
            kv.increment(m)
        del k, v
    for s, l in enumerate(lens0):
        kv.set_seq_len(l, seq=s)

    # Per-step inputs, resident before timing: one set per step (warmup reuses the first).
    n_sets = max(steps, 1)
    qs = [[torch.randn((B, n_head, hd), generator=gen, device=dev).mul_(sq) for _ in range(L)] for _ in range(n_sets)]
    ks = [[torch.randn((B, 1, n_kv, hd), generator=gen, device=dev).mul_(skv) for _ in range(L)] for _ in range(n_sets)]
    vs = [[torch.randn((B, 1, n_kv, hd), generator=gen, device=dev).mul_(skv) for _ in range(L)] for _ in range(n_sets)]
    out = torch.empty((B, n_head, hd), device=dev)
    ws = kv.workspace(n_head)
    torch.cuda.synchronize()

    fold = args.fold and not args.separate

    def step(i, events=None):
        for layer in range(L):
            if args.separate:
                kv.append_quant(layer, ks[i][layer], vs[i][layer], rope)
            if events is not None:
                events[layer][0].record()
            if args.separate:
                kv.attn_decode(layer, qs[i][layer], rope, out=out, workspace=ws)
            else:  # quantize_kv + main_attn_out_int4 in one launch; the last layer's launch
                # also advances the lengths (cache.increment()) unless --no-fold
                kv.attn_decode_append(layer, ks[i][layer], vs[i][layer], qs[i][layer], rope,
                                      out=out, workspace=ws, advance=fold and layer == L - 1)
            if events is not None:
                events[layer][1].record()
        if not (fold and not args.separate):
            kv.increment(1)

    def reset_lens():
        for s, l in enumerate(lens0):
            kv.set_seq_len(l, seq=s)

    # Kernel timing pass (no graph): HIP events around every ts_attn_decode launch.
    n_kt = min(steps, 16)
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(L)] for _ in range(n_kt)]
    for i in range(min(warmup, 2)):
        step(i % n_sets)
    reset_lens()
    for i in range(n_kt):
        step(i, ev[i])
    torch.cuda.synchronize()
    reset_lens()
    torch.cuda.synchronize()

    # The timed steps.  With graphs, each step (36 x (append, decode split, combine) + the
    # length increment) is captured once with its own split plan and replayed; device lengths
    # advance inside the graphs exactly as in eager execution.
    graphs = None
    if args.graph:
        # one graph per step (default), or per group of spg consecutive steps (--steps-per-graph:
        # the host's launch cost per graph then spreads over spg steps)
        graphs = []
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        for i0 in range(0, steps, spg):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=cap):
                for i in range(i0, min(i0 + spg, steps)):
                    step(i)
            graphs.append(gr)
        torch.cuda.synchronize()
        for i in range(-(-warmup // spg)):  # warm_steps steps
            graphs[i % len(graphs)].replay()
        torch.cuda.synchronize()
        reset_lens()
    else:
        for i in range(warmup):
            step(i % n_sets)
        reset_lens()
    torch.cuda.synchronize()

    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    launcher = None
    if graphs is None and args.host_loop == "c":
        # the timed steps as calls of the library's decode entry points from a compiled loop
        # (ts_probe_decode_steps), eager launches as a compiled host would issue them
        if args.separate or not fold:
            sys.exit("--host-loop c without graphs runs the fused, folded step only")
        from airframe_amd._lib import load as load_ts
        from airframe_amd.build import PROBE_PATH
        tl = load_ts()
        plib = ctypes.CDLL(PROBE_PATH)
        vp = ctypes.c_void_p
        plib.ts_probe_decode_steps.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               vp, vp, vp, ctypes.c_int, vp, vp, vp, ctypes.c_uint64, vp]
        arr = lambda ts_: (vp * (n_sets * L))(*[t.data_ptr() for row in ts_ for t in row])  # noqa: E731
        k_a, v_a, q_a = arr(ks), arr(vs), arr(qs)
        fmid = ctypes.cast(tl.ts_attn_decode_append, vp)
        flast = ctypes.cast(tl.ts_attn_decode_append_advance, vp)
        cur = vp(torch.cuda.current_stream().cuda_stream)
        launcher = lambda: plib.ts_probe_decode_steps(  # noqa: E731
            fmid, flast, kv.handle, L, steps, n_sets, k_a, v_a, q_a, n_head, rope.handle,
            vp(out.data_ptr()), vp(ws.data_ptr()), ws.numel(), cur)
    if graphs is not None and args.host_loop == "c":
        # every step's graph launched from a compiled loop (ts_probe_graph_launch)
        from airframe_amd.build import PROBE_PATH
        plib = ctypes.CDLL(PROBE_PATH)
        plib.ts_probe_graph_launch.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.c_void_p]
        execs = (ctypes.c_void_p * len(graphs))(*[gr.raw_cuda_graph_exec() for gr in graphs])
        cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        launcher = lambda: plib.ts_probe_graph_launch(execs, len(graphs), cur)  # noqa: E731
        assert launcher() == 0  # one untimed pass (the lengths are reset below)
        torch.cuda.synchronize()
        reset_lens()
        torch.cuda.synchronize()
    t_start.record()
    if launcher is not None:
        rc = launcher()
        if rc != 0:
            sys.exit(f"hipGraphLaunch failed: {rc}")
    elif graphs is not None:
        for gr in graphs:
            gr.replay()
    else:
        for i in range(steps):
            step(i)
    t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_step = total_ms / steps

    step_bytes = 0
    kern_bytes = []
    for i in range(steps):
        ctx = [l + i + 1 for l in lens0]
        b = attn_bytes(ctx, n_kv, n_head, hd, B)
        # the timed launch also does the append unless the two calls are separate
        kern_bytes.append(b if args.separate else b + append_bytes(B, n_kv, hd))
        step_bytes += L * (b + append_bytes(B, n_kv, hd))
    step_bytes /= steps
    result = dict(total_ms=total_ms, ms_step=ms_step, step_bytes=step_bytes)
    kt = [ev[i][l][0].elapsed_time(ev[i][l][1]) for i in range(n_kt) for l in range(L)]
    kb = [kern_bytes[i] for i in range(n_kt) for _ in range(L)]
    result["kernel_ms"] = float(np.mean(kt))
    result["kernel_bytes"] = float(np.mean(kb))
    result["kernel_timing"] = "HIP events around each decode launch, eager pass of 16 steps"
    # The decode launches alone (no length increment), captured once as a graph of the L
    # launches of step 0 and replayed: the average time per launch without the host's
    # issue gaps between launches (also when the timed steps run eagerly).  Every replay
    # appends the same token at the same position.
    reset_lens()
    kg = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    # at least 32 launches per graph (the layers repeated), so that a one-layer config's
    # replays measure the launches and not the host's graph launch
    n_copies = -(-32 // L)
    with torch.cuda.graph(kg, stream=cap):
        for _ in range(n_copies):
            for layer in range(L):
                if args.separate:
                    kv.attn_decode(layer, qs[0][layer], rope, out=out, workspace=ws)
                else:
                    kv.attn_decode_append(layer, ks[0][layer], vs[0][layer], qs[0][layer], rope,
                                          out=out, workspace=ws)
    torch.cuda.synchronize()
    for _ in range(3):
        kg.replay()
    n_rep = 20
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n_rep):
        kg.replay()
    e1.record()
    torch.cuda.synchronize()
    result["kernel_ms"] = e0.elapsed_time(e1) / (n_rep * L * n_copies)
    result["kernel_bytes"] = float(kern_bytes[0])
    result["kernel_timing"] = (f"HIP events around {n_rep} replays of a graph holding only the {L * n_copies} "
                               "decode launches of step 0" + (f" ({n_copies} copies of the {L} layers)" if n_copies > 1 else "")
                               + " (split and combine kernels; no length increment)")
    del kg

    cpu = None
    reset_lens()
    torch.cuda.synchronize()
    del graphs
    if not args.no_cpu:
        from oracle import oracle
        table = oracle.rope_table(max_seq, hd, cfg["theta"])
        # The oracle appends at lens0 (same token the GPU appended in timed step 0).
        t_mt, cores, t_st = cpu_baseline(kv, cfg, qs[0], ks[0], vs[0], lens0, max_seq, table,
                                         layers_mt=min(2, L), seqs_st=min(2, B), norms=norms)
        cpu = dict(step_s_mt=t_mt, cores=cores, step_s_st=t_st)
    return result, cpu


def run_prefill(args, cfg):
    import torch

    from airframe_amd.kv_cache import KVCache, RopeTable

    dev = torch.device("cuda:0")
    L, n_head, n_kv, hd, B = cfg["layers"], cfg["n_head"], cfg["n_kv"], cfg["hd"], cfg["batch"]
    C, NC = cfg["chunk"], cfg["n_chunks"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    max_seq = C * NC
    rope = RopeTable(max_seq, hd, cfg["theta"])
    kv = KVCache.new_int4(L, n_kv, hd, max_seq, B)
    qs = [[torch.randn((B, C, n_head, hd), generator=gen, device=dev) for _ in range(L)] for _ in range(NC)]
    ks = [[torch.randn((B, C, n_kv, hd), generator=gen, device=dev) for _ in range(L)] for _ in range(NC)]
    vs = [[torch.randn((B, C, n_kv, hd), generator=gen, device=dev) for _ in range(L)] for _ in range(NC)]
    out = torch.empty((B, C, n_head, hd), device=dev)

    def run(events=None):
        kv.reset()
        for c in range(NC):
            for layer in range(L):
                kv.append_quant(layer, ks[c][layer], vs[c][layer], rope)
                if events is not None:
                    events[c][layer][0].record()
                kv.attn_prefill(layer, qs[c][layer], rope, out=out)
                if events is not None:
                    events[c][layer][1].record()
            kv.increment(C)

    for _ in range(max(args.warmup, 1)):
        run()
    torch.cuda.synchronize()
    reps = max(args.steps, 1)
    # Per-launch prefill time: events around each eager prefill launch.
    evs = [[[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(L)] for _ in range(NC)] for _ in range(reps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for r in range(reps):
        run(evs[r])
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1) / reps
    kt = [evs[r][c][l][0].elapsed_time(evs[r][c][l][1]) for r in range(reps) for c in range(NC) for l in range(L)]
    launch = "eager"
    if args.graph:
        # The step (reset, then every chunk's appends, prefills and length increment) captured
        # once as a HIP graph and replayed: device lengths restart at 0 in every replay.
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=cap):
            run()
        torch.cuda.synchronize()
        for _ in range(2):
            gr.replay()
        torch.cuda.synchronize()
        t0.record()
        for r in range(reps):
            gr.replay()
        t1.record()
        torch.cuda.synchronize()
        total_ms = t0.elapsed_time(t1) / reps
        launch = "hip-graph replay per step"
    # causal-exact flops per layer: QK^T and PV, 2 flops per MAC, over all chunks
    n_tot = C * NC
    flops_layer = 4 * hd * n_head * B * (n_tot * (n_tot + 1) // 2)
    kernel_ms_layer = float(np.sum(kt)) / reps / L
    res = dict(total_ms=total_ms, kernel_ms_layer=kernel_ms_layer, flops_layer=flops_layer, launch=launch)
    if not args.no_cpu:
        res["cpu"] = cpu_baseline_prefill(cfg, qs, ks, vs)
    return res


def cpu_baseline_prefill(cfg, qs, ks, vs):
    """The C oracle on a bounded sample of config 5's layer: sequence 0 of layer 0, all chunks
    (append + causal attention), OpenMP over heads; and its first chunk single-threaded.  The
    rates are flops of the sample / its time (the same causal-exact counting as the GPU)."""
    from oracle import oracle
    n_head, n_kv, hd, C, NC = cfg["n_head"], cfg["n_kv"], cfg["hd"], cfg["chunk"], cfg["n_chunks"]
    threads = cpu_threads()
    table = oracle.rope_table(C * NC, hd, cfg["theta"])

    def run(n_chunks, thr):
        ora = oracle.OracleKV(1, C * NC, n_kv, hd, table)
        t = 0.0
        for c in range(n_chunks):
            k = ks[c][0][:1].cpu().numpy()
            v = vs[c][0][:1].cpu().numpy()
            q = qs[c][0][:1].cpu().numpy()
            t0 = time.perf_counter()
            ora.append(k, v)
            ora.attend(q, C, threads=thr)
            t += time.perf_counter() - t0
            ora.advance(C)
        n = n_chunks * C
        return 4 * hd * n_head * (n * (n + 1) // 2) / t / 1e12

    return dict(tflops_mt=run(NC, threads), cores=threads, tflops_st=run(1, 1))


def run_append(args, cfg):
    """Quantize-on-append of one 512-token prefill chunk per sequence (the configuration's
    batch, kv heads and head dim), every layer, cache empty before each chunk.  Returns the
    mean time of one ts_append_quant call and its algorithmic bytes: the f32 K and V read and
    the packed rows and scales written."""
    import torch

    from airframe_amd.kv_cache import KVCache, RopeTable

    dev = torch.device("cuda:0")
    L, n_kv, hd, B = cfg["layers"], cfg["n_kv"], cfg["hd"], cfg["batch"]
    n_tok = 512
    rope = RopeTable(n_tok + 8, hd, cfg["theta"])
    kv = KVCache.new_int4(L, n_kv, hd, n_tok + 8, B)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ks = [torch.randn((B, n_tok, n_kv, hd), generator=gen, device=dev) for _ in range(L)]
    vs = [torch.randn((B, n_tok, n_kv, hd), generator=gen, device=dev) for _ in range(L)]
    if args.qk_norm:
        for layer in range(L):
            kv.set_qk_norm(layer, None, torch.randn(hd, generator=gen, device=dev) * 0.2 + 1.0)
    for layer in range(L):
        kv.append_quant(layer, ks[layer], vs[layer], rope)
    torch.cuda.synchronize()
    reps = 5
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for layer in range(L):
            kv.append_quant(layer, ks[layer], vs[layer], rope)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * L)
    return ms, B * n_tok * n_kv * (2 * hd * 4 + hd + 8), B * n_tok


KQ_BLOCK = {12: 144, 13: 176, 8: 272, 2: 144, 6: 176}  # bytes of 256 elements of a Q4_K / Q5_K / Q8_0 / Q4_0 / Q5_0 row


def kq_blob(gen, rows, cols, ggml_type, dev):
    """Random GGUF blocks of an [rows][cols] matrix on the device: random bytes with finite f16
    scales (d and dmin of the K formats; d of every 32-element Q8_0 / Q4_0 block) of about 1e-4
    (weights of about 1e-2)."""
    import torch
    if ggml_type in (12, 13):
        nb = rows * cols // 256
        bb = KQ_BLOCK[ggml_type]
        b = torch.randint(0, 256, (nb, bb), generator=gen, device=dev, dtype=torch.uint8)
        dd = (torch.rand((nb, 2), generator=gen, device=dev) * 3e-4 + 1e-4).half()
        b[:, 0:4] = dd.view(torch.uint8).reshape(nb, 4)
        return b.reshape(-1)
    nb = rows * cols // 32
    bb = KQ_BLOCK[ggml_type] // 8
    b = torch.randint(0, 256, (nb, bb), generator=gen, device=dev, dtype=torch.uint8)
    dd = (torch.rand((nb, 1), generator=gen, device=dev) * 3e-4 + 1e-4).half()
    b[:, 0:2] = dd.view(torch.uint8).reshape(nb, 2)
    return b.reshape(-1)


def run_qkv(args, cfg):
    """The fused QKV projection + append (ts_qkv_append) of one step of the configuration:
    one token per sequence for the decode configurations, one 512-token chunk per sequence
    for config 5; every layer with its own f16 weights (so no layer's weights are still cached
    when it runs again).  Returns the mean time of one call, its algorithmic bytes (weights,
    x, q written, packed K/V rows and scales written) and its algorithmic flops (2 M N K)."""
    import torch

    from airframe_amd.kv_cache import KVCache, RopeTable

    dev = torch.device("cuda:0")
    L, n_head, n_kv, hd, B, dim = (cfg["layers"], cfg["n_head"], cfg["n_kv"], cfg["hd"],
                                   cfg["batch"], cfg["dim"])
    n_tok = cfg.get("chunk", 1)
    reps = 5 if n_tok == 1 else 2
    max_seq = n_tok * (reps + 3) + 8  # warmup, one untimed replay, reps replays
    rope = RopeTable(max_seq, hd, cfg["theta"])
    kv = KVCache.new_int4(L, n_kv, hd, max_seq, B)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    P = args.planes  # 2: rows of [hi dim | lo dim] (F32 / GGUF block weights, ts_qkv_append_x2)

    def w(rows):
        return (torch.randn((rows, P * dim), generator=gen, device=dev) * 0.02).half()

    T = CONVERT_TYPES[args.gguf] if args.gguf else None
    if T is not None:  # GGUF K-quant blocks read in the loop (ts_qkv_append_gguf)
        ws = [tuple(kq_blob(gen, r, dim, T, dev) for r in (n_head * hd, n_kv * hd, n_kv * hd)) for _ in range(L)]
        w_bytes_per = KQ_BLOCK[T] / 256
    else:
        ws = [(w(n_head * hd), w(n_kv * hd), w(n_kv * hd)) for _ in range(L)]
        w_bytes_per = 2 * P
    x = torch.randn((B, n_tok, dim), generator=gen, device=dev)
    q = torch.empty((B, n_tok, n_head, hd), device=dev)
    scratch = kv.qkv_workspace(dim, n_tok, n_head) if T is None else None
    if args.qk_norm:
        for layer in range(L):
            kv.set_qk_norm(layer, None, torch.randn(hd, generator=gen, device=dev) * 0.2 + 1.0)

    def call(layer):
        if T is not None:
            kv.qkv_append_gguf(layer, x, T, *ws[layer], rope, q_out=q)
        else:
            kv.qkv_append(layer, x, *ws[layer], rope, q_out=q, workspace=scratch, planes=P)

    for layer in range(L):
        call(layer)
    kv.increment(n_tok)
    torch.cuda.synchronize()
    # one step (every layer's call, then the length increment) captured as a graph and
    # replayed, so the time is the kernels' and not the host's launch loop
    gr = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(gr, stream=cap):
        for layer in range(L):
            call(layer)
        kv.increment(n_tok)
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * L)
    M, N = B * n_tok, (n_head + 2 * n_kv) * hd
    byts = int(N * dim * w_bytes_per) + M * dim * 4 + M * n_head * hd * 4 + M * n_kv * (hd + 8)
    return ms, byts, 2.0 * M * N * dim, M


CONVERT_TYPES = {"f32": 0, "q4_0": 2, "q5_0": 6, "q8_0": 8, "q4_k": 12, "q5_k": 13, "q6_k": 14}


def run_convert(args, cfg):
    """ts_weights_to_f16x2 on a matrix of the configuration's Wq shape [n_head hd, dim] holding
    random blocks of the chosen GGUF type (finite f16 scales).  Returns the mean time of one
    call (us), its algorithmic bytes (the GGUF bytes read, 4 bytes per element written), rows
    and cols."""
    import numpy as np
    import torch

    from airframe_amd import weights

    t = CONVERT_TYPES[args.convert]
    rows, cols = cfg["n_head"] * cfg["hd"], cfg["dim"]
    nbytes = weights.src_bytes(t, rows, cols)
    rng = np.random.default_rng(args.seed)
    blob = rng.integers(0, 256, nbytes, dtype=np.uint8)
    if t != 0:  # every f16 field that is a scale gets a finite value: rewrite the blocks' headers
        epb, bpb = {2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}[t]
        blk = blob.reshape(-1, bpb)
        sc = np.frombuffer(rng.uniform(1e-4, 1e-3, (blk.shape[0], 2)).astype(np.float16).tobytes(), np.uint8)
        sc = sc.reshape(-1, 4)
        if t == 14:
            blk[:, 208:210] = sc[:, 0:2]
        else:
            blk[:, 0:2] = sc[:, 0:2]
            if t in (12, 13):
                blk[:, 2:4] = sc[:, 2:4]
    else:
        blob = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32).view(np.uint8)
    src = torch.from_numpy(blob).cuda()
    for _ in range(3):
        out = weights.to_f16(t, src, rows, cols, planes=2)
    torch.cuda.synchronize()
    reps = 20
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        out = weights.to_f16(t, src, rows, cols, planes=2)
    e1.record()
    torch.cuda.synchronize()
    del out
    return e0.elapsed_time(e1) * 1e3 / reps, nbytes + rows * cols * 4, rows, cols


def run_proj(args, cfg):
    """The attention output projection with the residual add (ts_attn_out_proj) of one step:
    one token per sequence for the decode configurations, a 512-token chunk per sequence for
    config 5; every layer with its own f16 weights.  Returns the mean time of one call, its
    algorithmic bytes (weights, attention output, the residual read and written) and flops."""
    import torch

    from airframe_amd.kv_cache import attn_out_proj

    dev = torch.device("cuda:0")
    L, n_head, hd, B, dim = cfg["layers"], cfg["n_head"], cfg["hd"], cfg["batch"], cfg["dim"]
    M, K = B * cfg.get("chunk", 1), n_head * hd
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    from airframe_amd.kv_cache import attn_out_proj_gguf
    P = args.planes
    T = CONVERT_TYPES[args.gguf] if args.gguf else None
    if T is not None:
        ws = [kq_blob(gen, dim, K, T, dev) for _ in range(L)]
        w_bytes = dim * K * KQ_BLOCK[T] // 256
    else:
        ws = [(torch.randn((dim, P * K), generator=gen, device=dev) * 0.02).half() for _ in range(L)]
        w_bytes = dim * K * 2 * P
    a = torch.randn((M, K), generator=gen, device=dev)
    act = torch.randn((M, dim), generator=gen, device=dev)

    def call(layer):
        if T is not None:
            attn_out_proj_gguf(a, T, ws[layer], dim, act)
        else:
            attn_out_proj(a, ws[layer], act, planes=P)

    for layer in range(L):
        call(layer)
    torch.cuda.synchronize()
    reps = 5
    gr = torch.cuda.CUDAGraph()  # every layer's call as one graph, replayed
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(gr, stream=cap):
        for layer in range(L):
            call(layer)
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * L)
    return ms, w_bytes + M * K * 4 + M * dim * 8, 2.0 * M * dim * K, M


def run_compact(args, cfg):
    """Sliding-window compaction (ts_kv_shift) on a cache of the configuration's shape: every
    sequence of every layer filled to ctx, then each sequence compacted (keep_sink 4, shift
    ctx/2) layer by layer.  Returns the time of the shifts and the bytes they move: the moved
    slots' K/V words and scales read once and written once at their new slots (a shift of at
    least the moved count is one in-place round)."""
    import torch

    from airframe_amd.kv_cache import KVCache, RopeTable

    dev = torch.device("cuda:0")
    L, n_kv, hd, B, ctx = cfg["layers"], cfg["n_kv"], cfg["hd"], cfg["batch"], cfg["ctx"]
    rope = RopeTable(2 * ctx + 8, hd, cfg["theta"])
    kv = KVCache.new_int4(L, n_kv, hd, ctx + 8, B)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    for layer in range(L):
        kv.reset()
        for t0 in range(0, ctx, 1024):
            m = min(1024, ctx - t0)
            k = torch.randn((B, m, n_kv, hd), generator=gen, device=dev)
            kv.append_quant(layer, k, k, rope)
            kv.increment(m)
    keep, amt = 4, ctx // 2
    n_move = ctx - keep - amt
    ws = torch.empty(kv.max_len() * n_kv * (hd + 8), dtype=torch.uint8, device=dev)
    # warm-up shift on layer 0, sequence 0 (moves data, which is all this measures)
    kv.shift_int4(0, keep, amt, 0, workspace=ws)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for s in range(B):
        for layer in range(L):
            kv.shift_int4(layer, keep, amt, s, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    per = n_move * n_kv * (hd + 8)  # one (sequence, layer): the moved slots' bytes
    return ms, 2 * per * B * L, B * L


def run_mfma_rates(args):
    """Issue rates of the matrix-core instructions the attention kernels use
    (airframe_amd/csrc/ts_probe.hip): independent chains back to back on every SIMD, no
    memory traffic.  The prefill kernel runs q's low half as scaled fp6 MFMAs because of the
    ratio between the first two lines."""
    import ctypes
    import torch
    from airframe_amd.build import PROBE_PATH
    if not os.path.exists(PROBE_PATH):
        sys.exit(f"{PROBE_PATH} is missing: run python -m airframe_amd.build")
    lib = ctypes.CDLL(PROBE_PATH)
    sink = torch.zeros(4, dtype=torch.float32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    grid, iters = 2048, 2000
    names = {0: "f16 v_mfma_f32_32x32x16_f16", 1: "fp6 e2m3 v_mfma_scale_f32_32x32x64_f8f6f4",
             2: "fp8 e4m3 v_mfma_scale_f32_32x32x64_f8f6f4", 3: "fp6 x fp8 v_mfma_scale_f32_32x32x64_f8f6f4"}
    out = {}
    for kind, name in names.items():
        flops = (32768 if kind == 0 else 131072) * 4 * iters * grid * 4  # 4 waves, 4 chains
        for _ in range(2):
            assert lib.ts_probe_mfma_rate(kind, grid, iters, ctypes.c_void_p(sink.data_ptr()), st) == 0
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        assert lib.ts_probe_mfma_rate(kind, grid, iters, ctypes.c_void_p(sink.data_ptr()), st) == 0
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        out[name] = round(flops / (ms * 1e-3) / 1e12, 1)
    return {"metric": "matrix-core issue rate, TFLOP/s (dense, independent chains)", "rates": out,
            "n_gpus": 1, "grid": grid, "iters": iters, "config": {"workload": "mfma_rate_probe"},
            "data": "register operands, no memory traffic"}


def run_stream_ceiling(args, cfg):
    """HBM ceilings for the decode step's reads (airframe_amd/csrc/ts_probe.hip): the decode
    kernel's exact access pattern with no math (one launch reads what one layer's decode
    reads), and a flat grid-strided read of the same byte count.  Four distinct buffer sets,
    used round robin, so the 256 MB Infinity Cache cannot serve repeats."""
    import ctypes
    import torch
    from airframe_amd.build import PROBE_PATH
    if not os.path.exists(PROBE_PATH):
        sys.exit(f"{PROBE_PATH} is missing: run python -m airframe_amd.build")
    lib = ctypes.CDLL(PROBE_PATH)
    lib.ts_probe_flat_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_void_p]
    B, H, hd, ctx = cfg["batch"], cfg["n_kv"], cfg["hd"], cfg["ctx"] + 1
    P = (ctx + 63) // 64 * 64
    rows = B * H
    n_sets = 4
    sets = [(torch.empty(rows * P * hd // 2, dtype=torch.uint8, device="cuda"),
             torch.empty(rows * P * hd // 2, dtype=torch.uint8, device="cuda"),
             torch.empty(rows * P, dtype=torch.float32, device="cuda"),
             torch.empty(rows * P, dtype=torch.float32, device="cuda")) for _ in range(n_sets)]
    nbytes = rows * ctx * (hd + 8)
    flat = [torch.empty(nbytes // 16 * 16, dtype=torch.uint8, device="cuda") for _ in range(n_sets)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def timed(f, n):
        for i in range(3):
            f(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            f(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e3

    def dec(i, stamps=None):
        kp, vp, ks, vs = sets[i % n_sets]
        rc = lib.ts_probe_decode_loads(ctypes.c_void_p(kp.data_ptr()), ctypes.c_void_p(vp.data_ptr()),
                                       ctypes.c_void_p(ks.data_ptr()), ctypes.c_void_p(vs.data_ptr()),
                                       B, H, hd, P, ctx, ctypes.c_void_p(sink.data_ptr()),
                                       ctypes.c_void_p(stamps.data_ptr() if stamps is not None else 0), st)
        assert rc == 0, rc

    def flat_read(i):
        rc = lib.ts_probe_flat_read(ctypes.c_void_p(flat[i % n_sets].data_ptr()), nbytes // 16, 2048,
                                    ctypes.c_void_p(sink.data_ptr()), st)
        assert rc == 0, rc

    n = max(args.steps, 20)
    us_dec = timed(dec, n)
    us_flat = timed(flat_read, n)
    res = dict(bytes=nbytes, us_decode_pattern=us_dec, us_flat=us_flat, launches=n)

    # per-workgroup stamps of 8 launches (start and end of its loads, 100 MHz clock, and its
    # XCD): the per-XCD medians of the workgroups' streaming time and of their end times
    stamps = torch.zeros(3 * B * H, dtype=torch.int64, device="cuda")
    per_xcd, ends = {}, {}
    for i in range(8):
        dec(i, stamps)
        torch.cuda.synchronize()
        t = stamps.view(-1, 3).cpu().numpy()
        t0 = t[:, 0].min()
        for start, end, x in t:
            per_xcd.setdefault(int(x), []).append((end - start) * 0.01)  # us
            ends.setdefault(int(x), []).append((end - t0) * 0.01)
    med = {x: float(np.median(v)) for x, v in sorted(per_xcd.items())}
    res["per_xcd_median_stream_us"] = {str(x): round(v, 2) for x, v in med.items()}
    res["per_xcd_median_end_us"] = {str(x): round(float(np.median(v)), 2) for x, v in sorted(ends.items())}
    res["xcd_spread"] = round(max(med.values()) / min(med.values()), 4) if med else None

    # the same reads as 16-window units claimed from a launch-wide counter (a work queue)
    nw = ctx // 64 // 16 * 16
    if nw >= 16:
        ctr = torch.zeros(n + 8, dtype=torch.int32, device="cuda")  # one zeroed counter per launch
        used = [0]

        def claimed(i):
            kp, vp, ks, vs = sets[i % n_sets]
            slot = used[0]
            used[0] += 1
            rc = lib.ts_probe_claim_loads(ctypes.c_void_p(kp.data_ptr()), ctypes.c_void_p(vp.data_ptr()),
                                          ctypes.c_void_p(ks.data_ptr()), ctypes.c_void_p(vs.data_ptr()),
                                          B, H, hd, P, 64 * nw, 16, 256,
                                          ctypes.c_void_p(ctr.data_ptr() + 4 * slot),
                                          ctypes.c_void_p(sink.data_ptr()), st)
            assert rc == 0, rc

        ctr.zero_()
        res["us_claimed_units"] = timed(claimed, n) * ctx / (64 * nw)  # scaled to the same bytes
    # the per-launch cost of a kernel in a graph: 36 empty 256-workgroup launches, replayed
    gr = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(gr, stream=cap):
        for _ in range(36):
            lib.ts_probe_empty(256, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(cap.cuda_stream))
    gr.replay()
    torch.cuda.synchronize()
    res["us_empty_launch_in_graph"] = timed(lambda i: gr.replay(), 20) / 36
    return res


def _split_kernel_name(cfg, n_cu=256):
    """Which split kernel the library launches for this shape: decode_plan and the dispatch
    rule of launch_decode (ts_decode.hip), restated for the bench label (the step's starting
    lengths; MI355X has 256 CUs)."""
    if "ragged" in cfg:
        rng = np.random.default_rng(2024)
        ctx = [int(x) + 1 for x in rng.integers(cfg["ragged"][0], cfg["ragged"][1], size=cfg["batch"])]
    else:
        ctx = [cfg["ctx"] + 1] * cfg["batch"]

    def chunk_for(target):
        busy = lambda c: sum(-(-x // c) for x in ctx) * cfg["n_kv"]
        hi = max(256, -(-max(ctx) // 64) * 64)
        lo = min(hi, max(256, -(-sum(ctx) * cfg["n_kv"] // target)))
        lo = -(-lo // 64) * 64
        c = lo
        while c < hi and busy(c) > target:
            c += 64
        return lo if busy(c) > target else c  # no chunk meets the target: the balanced one

    stored = 64 if cfg["hd"] <= 64 else 128 if cfg["hd"] <= 128 else 256
    gmax = 16 if stored <= 128 else 8  # decode_int_gmax (ts_internal.h)
    g4 = cfg["n_head"] // cfg["n_kv"] <= gmax and chunk_for(n_cu - n_cu // 8) >= 1024
    return "decode_split4_kernel" if g4 else "decode_split_kernel"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIGS))
    ap.add_argument("--head-dim", type=int, default=None,
                    help="another head dim (e.g. 256, Gemma-2's), the workload renamed")
    ap.add_argument("--n-head", type=int, default=None, help="another query head count")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--separate", action="store_true",
                    help="decode: ts_append_quant + ts_attn_decode instead of the fused launch")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a plain 1 GiB device copy (4 launches) so rocprofv3 HBM counters "
                         "can be scaled by what they read for a copy of known size")
    ap.add_argument("--append", action="store_true",
                    help="measure quantize-on-append (ts_append_quant) of a 512-token chunk per "
                         "sequence at the config's shape instead of the decode step")
    ap.add_argument("--qk-norm", action="store_true",
                    help="turn on the fused Qwen3 QK norm (random weights) for the decode step or "
                         "the append measurement")
    ap.add_argument("--qkv", action="store_true",
                    help="time the fused QKV projection + append (ts_qkv_append) instead")
    ap.add_argument("--proj", action="store_true",
                    help="time the attention output projection + residual (ts_attn_out_proj) instead")
    ap.add_argument("--planes", type=int, default=1, choices=(1, 2),
                    help="with --qkv/--proj: 2 = two-plane weights (F32 / GGUF formats, the _x2 entry points)")
    ap.add_argument("--gguf", default=None, choices=("q4_k", "q5_k", "q8_0", "q4_0", "q5_0"),
                    help="with --qkv/--proj: weights as GGUF blocks read in the loop (the _gguf entry points)")
    ap.add_argument("--convert", default=None, choices=sorted(CONVERT_TYPES),
                    help="time ts_weights_to_f16x2 on the configuration's Wq of that GGUF type")
    ap.add_argument("--compact", action="store_true",
                    help="measure sliding-window compaction (ts_kv_shift) on the config's cache "
                         "instead of the decode step")
    ap.add_argument("--mfma-rates", action="store_true",
                    help="matrix-core issue rates of f16 and scaled fp6/fp8 MFMAs (ts_probe.hip)")
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="measure the HBM ceiling of the decode's access pattern with no math "
                         "(loads-only probe at the config's shape) and of a flat read of the same size")
    ap.add_argument("--host-loop", default="auto", choices=("auto", "python", "c"),
                    help="who issues the timed decode steps: Python (graph replays, or the KVCache "
                         "methods with --no-graph) or a compiled loop (hipGraphLaunch of the step "
                         "graphs, or with --no-graph the library's C entry points, as a compiled "
                         "host calls them: ts_probe_graph_launch / ts_probe_decode_steps); auto: "
                         "the compiled loop of library calls for the batch-1 configurations 1 and 2, "
                         "whose steps are short enough for the host's issue cost to show, else "
                         "Python graph replays")
    ap.add_argument("--steps-per-graph", type=int, default=1,
                    help="decode: capture this many consecutive steps per HIP graph (default 1: one graph per step)")
    ap.add_argument("--no-fold", dest="fold", action="store_false",
                    help="decode: a separate length-update launch per step instead of the last layer's "
                         "ts_attn_decode_append_advance")
    ap.add_argument("--no-graph", dest="graph", action="store_false",
                    help="launch every kernel eagerly instead of replaying captured HIP graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the INT4 KV path shards "
                          "by sequence or kv head with no exchange, but "
                          "multi-GPU runs are not part of it", "n_gpus": args.gpus}))
        sys.exit(2)
    cfg = dict(CONFIGS[args.config])
    if args.head_dim or args.n_head:
        cfg["hd"] = args.head_dim or cfg["hd"]
        cfg["n_head"] = args.n_head or cfg["n_head"]
        cfg["name"] += f"_hd{cfg['hd']}_h{cfg['n_head']}"
    if args.steps is None:
        args.steps = cfg.get("steps", 3) if args.config != 5 else 3
    if args.host_loop == "auto":
        if args.config in (1, 2) and args.fold and not args.separate and args.steps_per_graph <= 1:
            args.host_loop, args.graph = "c", False
        else:
            args.host_loop = "python"

    import torch
    import airframe_amd
    airframe_amd.load()
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    torch.cuda.set_device(0)
    if args.append:
        if "ctx" not in cfg:
            sys.exit("--append needs a decode configuration (1-4)")
        ms, byts, toks = run_append(args, cfg)
        gbs = byts / (ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": "INT4 KV quantize-on-append HBM GB/s", "value": round(gbs, 1), "unit": "GB/s",
            "n_gpus": 1, "higher_is_better": True, "us_per_call": round(ms * 1e3, 2),
            "tokens_per_s": round(toks / (ms * 1e-3), 1),
            "config": {"workload": cfg["name"] + "_append_512tok" + ("_qknorm" if args.qk_norm else ""),
                       "tokens_per_call": toks},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_call": byts,
                         "counting": "f32 K and V read, packed K/V rows and two scales written"},
            "data": "synthetic"}), flush=True)
        return
    if args.convert:
        us, byts, rows, cols = run_convert(args, cfg)
        gbs = byts / (us * 1e-6) / 1e9
        print(json.dumps({
            "metric": f"GGUF {args.convert} weight conversion to two f16 planes GB/s", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "us_per_call": round(us, 2),
            "config": {"workload": f"{cfg['name']}_wq_{args.convert}", "rows": rows, "cols": cols},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": byts,
                         "counting": "GGUF bytes read, two f16 planes written"},
            "data": "synthetic (random blocks, finite scales)"}), flush=True)
        return
    if args.qkv or args.proj:
        ms, byts, flops, toks = (run_qkv if args.qkv else run_proj)(args, cfg)
        what = "fused QKV projection + INT4 append" if args.qkv else "attention output projection + residual"
        decode = "ctx" in cfg
        gbs = byts / (ms * 1e-3) / 1e9
        tfs = flops / (ms * 1e-3) / 1e12
        roof = ({"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                 "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": byts,
                 "counting": (("GGUF block bytes" if args.gguf else "f16 weights (both planes with --planes 2)")
                              + (" and f32 x read, f32 q, packed K/V rows and scales written" if args.qkv
                                 else " and f32 attention output read, residual read and written"))}
                if decode else
                {"bound": "mfma", "achieved": round(tfs, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                 "unit": "TFLOP/s", "frac": round(tfs / MFMA_F16_PEAK_TFLOPS, 4),
                 "flops_per_call": flops, "counting": "2 M N K of the projection (the hi/lo split "
                 "of x executes twice that on the matrix cores)"})
        print(json.dumps({
            "metric": what + (" HBM GB/s" if decode else " TFLOP/s"),
            "value": round(gbs if decode else tfs, 2), "unit": "GB/s" if decode else "TFLOP/s",
            "n_gpus": 1, "higher_is_better": True, "us_per_call": round(ms * 1e3, 2),
            "tokens_per_s": round(toks / (ms * 1e-3), 1),
            "config": {"workload": cfg["name"] + ("_qkv" if args.qkv else "_oproj") + ("_qknorm" if args.qk_norm else "")
                       + ("_x2" if args.planes == 2 and not args.gguf else "")
                       + (f"_{args.gguf}_in_loop" if args.gguf else ""),
                       "tokens_per_call": toks, "dim": cfg["dim"]},
            "roofline": roof,
            "data": ("synthetic (random GGUF blocks, f16 scales ~1e-4, N(0,1) x)" if args.gguf
                     else "synthetic (random f16 weights, N(0,1) x)")}), flush=True)
        return
    if args.mfma_rates:
        print(json.dumps(run_mfma_rates(args)), flush=True)
        return
    if args.stream_ceiling:
        if "ctx" not in cfg or "ragged" in cfg:
            sys.exit("--stream-ceiling needs a uniform decode configuration (1-3)")
        r = run_stream_ceiling(args, cfg)
        g_dec = r["bytes"] / (r["us_decode_pattern"] * 1e-6) / 1e9
        g_flat = r["bytes"] / (r["us_flat"] * 1e-6) / 1e9
        print(json.dumps({
            "metric": "HBM streaming ceiling of the decode access pattern (loads only) GB/s",
            "value": round(g_dec, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "us_per_launch": round(r["us_decode_pattern"], 2), "frac": round(g_dec / HBM_PEAK_GBS, 4),
            "flat_read": {"GBps": round(g_flat, 1), "us_per_launch": round(r["us_flat"], 2),
                          "frac": round(g_flat / HBM_PEAK_GBS, 4)},
            "claimed_units_us_per_launch": round(r["us_claimed_units"], 2) if "us_claimed_units" in r else None,
            "empty_launch_in_graph_us": round(r["us_empty_launch_in_graph"], 2),
            "per_xcd_median_stream_us": r["per_xcd_median_stream_us"],
            "per_xcd_median_end_us": r["per_xcd_median_end_us"],
            "xcd_spread": r["xcd_spread"],
            "bytes_per_launch": r["bytes"], "launches": r["launches"],
            "config": {"workload": cfg["name"] + "_loads_only"}, "data": "uninitialised device buffers"}),
            flush=True)
        return
    if args.compact:
        if "ctx" not in cfg:
            sys.exit("--compact needs a decode configuration (1-4)")
        ms, moved, calls = run_compact(args, cfg)
        gbs = moved / (ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": "INT4 KV sliding-window compaction HBM GB/s", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "ms_total": round(ms, 3), "us_per_shift": round(ms * 1e3 / calls, 2),
            "config": {"workload": cfg["name"] + "_compact_keep4_shift_half", "shifts": calls},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_shift": moved // calls,
                         "counting": "moved slots' K/V words + scales: read once, written once "
                                     "at the new slots (2x)"},
            "data": "synthetic"}), flush=True)
        return
    # HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE (copy-calibrated) for
    # this configuration, as recorded in its profile summary; null when none was taken.
    traffic = traffic_commit = rocprof_us = None
    tpath = os.path.join(ROOT, "profiles", f"decode_cfg{args.config}.md")
    if os.path.exists(tpath) and not (args.head_dim or args.n_head):  # that profile's own workload
        with open(tpath) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    traffic = int(float(line.split(":")[1]))
                elif line.startswith("traffic_measured_at_commit:"):
                    traffic_commit = line.split(":", 1)[1].strip()
                elif line.startswith("rocprof_avg_us_per_launch:"):
                    rocprof_us = float(line.split(":")[1])

    if args.copy_calib:
        x = torch.empty(2**28, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(4):
            y.copy_(x)
        torch.cuda.synchronize()
        del x, y

    if args.config == 5:
        r = run_prefill(args, cfg)
        achieved = r["flops_layer"] / (r["kernel_ms_layer"] * 1e-3) / 1e12
        line = {
            "metric": "INT4-KV chunked-prefill attention MFMA TFLOP/s (% of f16 dense peak)",
            "value": round(r["flops_layer"] * cfg["layers"] / (r["total_ms"] * 1e-3) / 1e12, 3),
            "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r["total_ms"], 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int4-kv; f16 mfma (q and p*s_v high halves, p*s_v low half) + fp6 mfma (q low half, two terms)", "data": "synthetic",
            "launch": r["launch"],
            "config": {"workload": cfg["name"], "global_batch": cfg["batch"],
                       "seq_len": cfg["chunk"] * cfg["n_chunks"], "parallelism": "none"},
            "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                         "avg_launch_us": round(r["kernel_ms_layer"] * 1e3 / cfg["n_chunks"], 2),
                         "timing": (f"HIP events around each eager prefill launch ({cfg['n_chunks']} chunks x "
                                    f"{cfg['layers']} layers per step); avg_launch_us over all chunks")},
            "cpu_baseline": None if "cpu" not in r else {
                "value": round(r["cpu"]["tflops_mt"], 6), "unit": "TFLOP/s", "cores": r["cpu"]["cores"],
                "kind": "port", **cpu_info(),
                "single_thread_value": round(r["cpu"]["tflops_st"], 6),
                "sample": "C oracle: sequence 0 of layer 0, 4 chunks x 512 (append + causal "
                          f"attention, OpenMP over heads, {r['cpu']['cores']} threads); its first "
                          "chunk single-threaded; rates in the same causal-exact flops"},
        }
        print(json.dumps(line), flush=True)
        return

    r, cpu = run_decode(args, cfg)
    B, L = cfg["batch"], cfg["layers"]
    gbs = r["step_bytes"] / (r["ms_step"] * 1e-3) / 1e9
    tok_s = B / (r["ms_step"] * 1e-3)
    ach = r["kernel_bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
    split_name = _split_kernel_name(cfg)
    roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_source": (f"profiles/decode_cfg{args.config}.md (rocprofv3 --pmc FETCH_SIZE / "
                               f"WRITE_SIZE at commit {traffic_commit})") if traffic else None,
            "kernel": (f"{split_name}<{cfg['hd']}> (+ decode_combine_kernel when the plan splits; ts_attn_decode)"
                       if args.separate else
                       f"{split_name}<{cfg['hd']}> with fused append (+ decode_combine_kernel when the plan splits; ts_attn_decode_append)"),
            "bytes_per_launch": int(r["kernel_bytes"]),
            "avg_launch_us": round(r["kernel_ms"] * 1e3, 2),
            "timing": r["kernel_timing"]}
    if rocprof_us and not args.separate:
        # the same launch as rocprofv3 --kernel-trace times it (every dispatch on its own), from
        # the profile that also gives the traffic
        roof["rocprof_avg_launch_us"] = rocprof_us
        roof["rocprof_frac"] = round(r["kernel_bytes"] / (rocprof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    cpu_line = None
    if cpu:
        cpu_gbs = r["step_bytes"] / cpu["step_s_mt"] / 1e9
        cpu_line = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": cpu["cores"],
                    "kind": "port", **cpu_info(),
                    "tokens_per_s": round(B / cpu["step_s_mt"], 4),
                    "single_thread_tokens_per_s": round(B / cpu["step_s_st"], 5),
                    "sample": f"C oracle: append + attention of step 0 for all {B} sequences of "
                              f"2 layers (OpenMP, {cpu['cores']} threads), and of 2 sequences of "
                              f"1 layer single-threaded; scaled to {L} layers x {B} sequences"}
    line = {
        "metric": "INT4-KV decode-attn HBM GB/s (% of peak) + tokens/s, 8B shape ctx 8K b32",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["ms_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("int4-kv/f32-io (i8 mfma QK^T exact, f16 hi/lo PV)" if split_name == "decode_split4_kernel"
                  else "int4-kv/f32-io (f16 mfma, hi/lo split)"),
        "data": "synthetic (seeded N(0,1), x8 outlier channels)" if cfg["outliers"] else "synthetic (seeded N(0,1))",
        "tokens_per_s": round(tok_s, 1), "hbm_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "launch": (("eager" if not args.graph else "hip-graph replay per step" if args.steps_per_graph <= 1
                    else f"hip-graph replay per {args.steps_per_graph} steps")
                   + ((", graphs launched from a compiled loop" if args.graph else
                       ", library calls from a compiled loop") if args.host_loop == "c" else "")),
        "config": {"workload": cfg["name"] + ("_qknorm" if args.qk_norm else ""), "global_batch": B,
                   "seq_len": cfg.get("ctx"),
                   "layers": L, "n_head": cfg["n_head"], "n_head_kv": cfg["n_kv"],
                   "head_dim": cfg["hd"], "parallelism": "none"},
        "roofline": roof,
        "cpu_baseline": cpu_line,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
