"""CPU-side checks of the C ABI: the library loads, exports exactly what include/turboshimmy.h
declares, and its host-only entry points (RoPE table, sizing, argument validation) behave.
No GPU is touched here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import airframe_amd
from airframe_amd import _lib
from oracle import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "turboshimmy.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ts_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    L = airframe_amd.load()
    names = declared_functions()
    assert len(names) >= 19
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (ts_[a-z0-9_]+)$", out, flags=re.M))
    assert exported == set(names)


def _param_counts_c():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(ts_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text):
        args = " ".join(args.split())
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_integration_rust_block_matches_header():
    """The Rust extern block a maintainer would paste declares every C entry point, with the
    same number of arguments."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}")]
    rust = {}
    for name, args in re.findall(r"pub fn (ts_[a-z0-9_]+)\(([^)]*)\)", block, flags=re.S):
        args = " ".join(args.split()).rstrip(",")
        rust[name] = 0 if not args else args.count(",") + 1
    c = _param_counts_c()
    assert set(c) == set(declared_functions())
    assert set(rust) == set(c), sorted(set(rust) ^ set(c))
    assert rust == c, {k: (rust[k], c[k]) for k in c if rust[k] != c[k]}


def test_header_compiles_as_c():
    src = f'#include "{HEADER}"\nint main(void){{ ts_kv_desc d = {{1,1,1,64,1}}; (void)d; return 0; }}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-x", "c", "-", "-fsyntax-only"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


HEADER_HPP = os.path.join(os.path.dirname(HEADER), "turboshimmy.hpp")


def test_cpp_host_side_header_compiles():
    """include/turboshimmy.hpp (the C++ mirror of kv_cache.rs's KVCache) compiles as C++17
    with every member used."""
    src = f"""#include "{HEADER_HPP}"
namespace t = turboshimmy;
int use(t::KVCache &kv, t::RopeTable &r, float *p, unsigned *u, void *ws) {{
    kv.append_quant(0, p, p, 1, r); kv.requant_all(0, p, p, 1, 1, &r);
    kv.attn_decode(0, p, 8, r, p, ws, 0); kv.attn_decode_append(0, p, p, p, 8, r, p, ws, 0, true);
    kv.attn_prefill(0, p, 8, 1, r, p); kv.shift_int4(0, 4, 8, 0, ws, 0); kv.set_qk_norm(0, p, p);
    kv.export_layer(0, 0, 0, 1, u, u, p, p); kv.reset(); kv.reset(0, nullptr); kv.set_seq_len(1);
    kv.advance_window_base(1); t::Status s = kv.increment();
    return (int)kv.get_seq_len() + (int)kv.max_len() + (int)kv.get_window_base() + (int)kv.is_int4() +
           (int)kv.calculate_offset(0, 0, 0) + (int)kv.decode_workspace_bytes(8) + (int)kv.shift_workspace_bytes() +
           s.code + r.n_pos() + r.rope_dim() + (r.device_table() != nullptr);
}}
"""
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-x", "c++", "-", "-fsyntax-only"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_host_side_host_only_calls(tmp_path):
    """The C++ mirror's host-only members against the library on the CPU: the RoPE host
    table equals the oracle's bit for bit, bytes_for equals ts_kv_bytes, and a head_dim that
    is not a multiple of 8 is refused with an Error carrying TS_ERR_INVALID."""
    from oracle import oracle
    src = f"""#include "{HEADER_HPP}"
#include <cstdio>
int main() {{
    const auto t = turboshimmy::RopeTable::host_table(40, 64, 500000.0f);
    std::fwrite(t.data(), sizeof(float), t.size(), stdout);
    std::fprintf(stderr, "%llu\\n", (unsigned long long)turboshimmy::KVCache::bytes_for(2, 8, 128, 100, 3));
    try {{ (void)turboshimmy::KVCache::bytes_for(1, 8, 60, 16); }}
    catch (const turboshimmy::Error &e) {{ std::fprintf(stderr, "%d\\n", e.code()); }}
    return 0;
}}
"""
    exe = tmp_path / "host_only"
    libdir = os.path.dirname(_lib.LIB_PATH)
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-x", "c++", "-", "-o", str(exe),
                        f"-L{libdir}", "-lturboshimmy", f"-Wl,-rpath,{libdir}"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer(r.stdout, dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), oracle.rope_table(40, 64, 500000.0).reshape(-1).view(np.uint32))
    lines = r.stderr.decode().split()
    want = ctypes.c_uint64()
    d = _lib.KvDesc(2, 3, 8, 128, 100)
    assert airframe_amd.load().ts_kv_bytes(ctypes.byref(d), ctypes.byref(want)) == 0
    assert int(lines[0]) == want.value
    assert int(lines[1]) == _lib.TS_ERR_INVALID


def test_status_strings():
    L = airframe_amd.load()
    assert L.ts_status_string(0) == b"ok"
    assert b"overflow" in L.ts_status_string(_lib.TS_ERR_OVERFLOW)


@pytest.mark.parametrize("n_pos,rope_dim,base,scale,alpha,beta", [
    (600, 64, 500000.0, 1.0, 0.0, 0.0), (300, 128, 1000000.0, 1.0, 1.0, 32.0), (50, 128, 10000.0, 4.0, 0.0, 0.0),
    (9000, 128, 500000.0, 1.0, 0.0, 0.0),
    (700, 64, 10000.0, 0.5, 0.0, 0.0),           # linear (no YaRN parameters)
    (8192, 128, 500000.0, 0.25, 1.0, 32.0),      # YaRN, the spec defaults
    (4000, 4, 1.0001, 0.5, 0.1, 1.0),            # YaRN, preflight.rs:304-331's spec
    (3001, 96, 1000000.0, 0.3, 2.0, 16.0)])
def test_host_rope_table_bit_exact_with_oracle(n_pos, rope_dim, base, scale, alpha, beta):
    from airframe_amd.kv_cache import RopeTable
    t = RopeTable.host_table(n_pos, rope_dim, base, scale, alpha, beta)
    ref = oracle.rope_table(n_pos, rope_dim, base, scale, alpha, beta)
    assert np.array_equal(t.view(np.uint32), ref.view(np.uint32))


def test_host_rope_table_rejects_bad_args():
    L = airframe_amd.load()
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data_as(ctypes.c_void_p)
    assert L.ts_rope_table_host(p, 4, 7, 10000.0, 1.0) == _lib.TS_ERR_INVALID
    assert L.ts_rope_table_host(p, 4, 8, 10000.0, 0.0) == _lib.TS_ERR_INVALID
    assert L.ts_rope_table_host(p, 4, 8, 10000.0, float("nan")) == _lib.TS_ERR_INVALID
    assert L.ts_rope_table_host_yarn(p, 4, 8, 10000.0, -0.5, 1.0, 32.0) == _lib.TS_ERR_INVALID
    assert L.ts_rope_table_host_yarn(p, 4, 8, 10000.0, 0.5, 1.0, 32.0) == 0
    assert L.ts_rope_table_host(None, 4, 8, 10000.0, 1.0) == _lib.TS_ERR_INVALID


def test_kv_bytes_sizing():
    from airframe_amd.kv_cache import KVCache
    # Qwen3-8B shape, 36 layers, 32 sequences of 8192+128: packed K+V (hd/2 each) + 2 f32 scales
    b = KVCache.bytes_for(36, 8, 128, 8192 + 128, 32)
    P = (8192 + 128 + 63) // 64 * 64
    assert b == 36 * 32 * 8 * P * (64 + 64 + 4 + 4)
    assert b < 288e9
    # 7.5x smaller than the f32 cache the reference also allocates (kv_cache.rs:121-145)
    assert abs((36 * 32 * 8 * P * 128 * 4 * 2) / b - 7.53) < 0.01


def test_create_validates_before_touching_the_device():
    L = airframe_amd.load()
    h = ctypes.c_void_p()
    bad = [(0, 1, 1, 64, 16), (1, 1, 1, 60, 16), (1, 0, 1, 64, 16), (1, 1, 1, 64, 0)]
    for d in bad:
        assert L.ts_kv_create(ctypes.byref(_lib.KvDesc(*d)), ctypes.byref(h)) == _lib.TS_ERR_INVALID
    # a multiple of 8 past the largest stored head dim (the reference accepts any multiple of 8)
    assert L.ts_kv_create(ctypes.byref(_lib.KvDesc(1, 1, 1, 264, 16)), ctypes.byref(h)) == _lib.TS_ERR_UNSUPPORTED
    b = ctypes.c_uint64()
    assert L.ts_kv_bytes(ctypes.byref(_lib.KvDesc(1, 1, 1, 264, 16)), ctypes.byref(b)) == _lib.TS_ERR_UNSUPPORTED
    # other head dims up to 256 are stored padded to 64 / 128 / 256 dims
    assert L.ts_kv_bytes(ctypes.byref(_lib.KvDesc(2, 3, 4, 96, 100)), ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 2 * 3 * 4 * 128 * (128 + 8)
    assert L.ts_kv_bytes(ctypes.byref(_lib.KvDesc(1, 1, 1, 8, 64)), ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 64 * (64 + 8)
    assert L.ts_kv_bytes(ctypes.byref(_lib.KvDesc(1, 1, 1, 200, 64)), ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 64 * (256 + 8)
    assert L.ts_kv_create(None, ctypes.byref(h)) == _lib.TS_ERR_INVALID
    # null handles are rejected everywhere
    assert L.ts_kv_increment(None, 1, None) == _lib.TS_ERR_INVALID
    assert L.ts_attn_decode(None, 0, None, 32, None, 0.0, None, None, 0, None) == _lib.TS_ERR_INVALID
    assert L.ts_append_quant(None, 0, None, None, 1, None, None) == _lib.TS_ERR_INVALID


def test_out_proj_workspace_sizing_and_validation():
    """ts_attn_out_proj_workspace is host-only: the split partials for decode-sized batches,
    nothing for prefill tiles or unsplittable reductions, and argument checks."""
    L = airframe_amd.load()
    b = ctypes.c_uint64()
    # decode batch 32 at attn_dim 4096 -> dim 4096: 16 column tiles of 256, one 32-row tile,
    # the reduction split into slices of 256 (16 splits) -> 16 * 16 * 32 * 256 f32
    assert L.ts_attn_out_proj_workspace(32, 4096, 4096, ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 16 * 16 * 32 * 256 * 4
    assert L.ts_attn_out_proj_workspace(2048, 4096, 2560, ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 0                       # 64-row tiles over all of attn_dim
    assert L.ts_attn_out_proj_workspace(4, 320, 200, ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 0                       # 320 is not a multiple of 256: no split
    assert L.ts_attn_out_proj_workspace(0, 4096, 4096, ctypes.byref(b)) == _lib.TS_OK
    assert b.value == 0
    assert L.ts_attn_out_proj_workspace(4, 100, 64, ctypes.byref(b)) == _lib.TS_ERR_INVALID
    assert L.ts_attn_out_proj_workspace(4, 128, 64, None) == _lib.TS_ERR_INVALID
    assert L.ts_attn_out_proj(None, 1, 128, None, 64, None, None, None, 0, None) == _lib.TS_ERR_INVALID
    assert L.ts_qkv_workspace(None, 4096, 1, 32, ctypes.byref(b)) == _lib.TS_ERR_INVALID
    assert L.ts_qkv_append(None, 0, None, 4096, 1, None, None, None, 32, None, None, None, None,
                           None, 0, None) == _lib.TS_ERR_INVALID


def test_weights_src_bytes():
    """GGUF block sizes of the projection weight formats (elements, bytes per block:
    src/core/dequant/ and ggml_types.rs), host only."""
    L = airframe_amd.load()
    b = ctypes.c_uint64()
    shapes = {0: (1, 4), 1: (1, 2), 2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144), 13: (256, 176),
              14: (256, 210)}
    for t, (epb, bpb) in shapes.items():
        assert L.ts_weights_src_bytes(t, 3, 512, ctypes.byref(b)) == 0
        assert b.value == 3 * 512 // epb * bpb
    assert L.ts_weights_src_bytes(12, 3, 300, ctypes.byref(b)) == _lib.TS_ERR_INVALID   # partial block
    assert L.ts_weights_src_bytes(3, 3, 512, ctypes.byref(b)) == _lib.TS_ERR_UNSUPPORTED  # Q4_1
    assert L.ts_weights_src_bytes(8, 0, 512, ctypes.byref(b)) == _lib.TS_ERR_INVALID


def test_out_proj_workspace_covers_both_weight_layouts():
    L = airframe_amd.load()
    b = ctypes.c_uint64()
    assert L.ts_attn_out_proj_workspace(1, 4096, 4096, ctypes.byref(b)) == 0
    assert b.value > 0  # one token: the reduction is split
    assert L.ts_attn_out_proj_workspace(0, 4096, 4096, ctypes.byref(b)) == 0 and b.value == 0
