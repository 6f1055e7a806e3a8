"""Shared helpers of the GPU parity tests: drive the HIP path and the oracle on the same
seeded inputs and compare them to the stated bars."""
from __future__ import annotations

import sys

import numpy as np
import torch

from airframe_amd.kv_cache import KVCache, RopeTable
from oracle import oracle

# Attention outputs: |gpu - cpu| <= ATOL + RTOL * |cpu| elementwise (max-abs 2e-3 / rel 1e-3).
ATOL, RTOL = 2e-3, 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def assert_close(gpu: np.ndarray, ref: np.ndarray, what: str = ""):
    err = np.abs(gpu.astype(np.float64) - ref.astype(np.float64))
    bound = ATOL + RTOL * np.abs(ref.astype(np.float64))
    bad = ~(err <= bound)
    say(f"  {what}: max_abs_err={err.max():.3e} max_rel={np.max(err / (np.abs(ref) + 1e-30)):.3e} "
        f"violations={int(bad.sum())}")
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside {ATOL}+{RTOL}*|ref| (max err {err.max()})"


class Pair:
    """The GPU cache and the oracle cache, fed identical inputs."""

    def __init__(self, n_seq, n_kv, hd, max_seq, base, n_layers=1, rope_n_pos=None, rope_dim=None,
                 rope_scale=1.0, yarn=(0.0, 0.0)):
        self.n_seq, self.n_kv, self.hd = n_seq, n_kv, hd
        n_pos = rope_n_pos or max_seq
        rd = rope_dim or hd
        self.rope = RopeTable(n_pos, rd, base, rope_scale, *yarn)
        self.gpu = KVCache.new_int4(n_layers, n_kv, hd, max_seq, n_seq)
        self.ora = oracle.OracleKV(n_seq, max_seq, n_kv, hd, oracle.rope_table(n_pos, rd, base, rope_scale, *yarn))

    def append(self, k, v, layer=0):
        self.gpu.append_quant(layer, dev(k), dev(v), self.rope)
        self.ora.append(k, v)

    def advance(self, n):
        self.gpu.increment(n)
        self.ora.advance(n)

    def set_lens(self, lens):
        for s, l in enumerate(lens):
            self.gpu.set_seq_len(int(l), seq=s)
        self.ora.lens[:] = np.asarray(lens, np.int32)

    def check_codes(self, layer=0, upto=None):
        """Every written position, every sequence: packed words and scales bit-exact."""
        torch.cuda.synchronize()
        for s in range(self.n_seq):
            n = int(upto[s]) if upto is not None else int(self.ora.lens[s])
            if n == 0:
                continue
            kp, vp, ks, vs = self.gpu.export(layer, s, 0, n)
            kp = kp.cpu().numpy().view(np.uint32)
            vp = vp.cpu().numpy().view(np.uint32)
            ks = ks.cpu().numpy()
            vs = vs.cpu().numpy()
            for name, g, r in (("k_packed", kp, self.ora.k_packed[s, :n]), ("v_packed", vp, self.ora.v_packed[s, :n])):
                if not np.array_equal(g, r):
                    idx = np.argwhere(g != r)[0]
                    raise AssertionError(f"seq {s} {name} differs at {idx}: gpu {g[tuple(idx)]:#010x} cpu {r[tuple(idx)]:#010x}")
            for name, g, r in (("k_scale", ks, self.ora.k_scale[s, :n]), ("v_scale", vs, self.ora.v_scale[s, :n])):
                gb, rb = g.view(np.uint32), r.view(np.uint32)
                if not np.array_equal(gb, rb):
                    idx = np.argwhere(gb != rb)[0]
                    raise AssertionError(f"seq {s} {name} differs at {idx}: gpu {g[tuple(idx)]!r} cpu {r[tuple(idx)]!r}")
