"""Build libturboshimmy.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m airframe_amd.build

Objects go to airframe_amd/lib/obj, the library to airframe_amd/lib/libturboshimmy.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIBDIR, "libturboshimmy.so")
# bench.py --stream-ceiling's probes (not part of the C ABI)
PROBE_PATH = os.path.join(LIBDIR, "libts_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Files whose arithmetic must round exactly like the CPU reference get no FMA contraction.
EXACT = ["-ffp-contract=off"]

# MFMA accumulators in VGPRs: the attention kernels rescale them with VALU ops, which would
# otherwise cost two AGPR<->VGPR moves per accumulator register and window.
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]

SOURCES = {
    "ts_kv.cpp": EXACT,
    "ts_append.hip": EXACT,
    "ts_decode.hip": MFMA_VGPR,
    "ts_prefill.hip": MFMA_VGPR,
    "ts_qkv.hip": EXACT,
    "ts_proj.hip": EXACT,
    "ts_weights.hip": EXACT,
}
HEADERS = ["ts_internal.h", "ts_mfma.h", "ts_quant.h", "ts_store.h", "ts_gemm.h", "ts_kquant.h", os.path.join("..", "..", "include", "turboshimmy.h")]


def _compile(src: str, extra: list[str], objdir: str) -> str:
    obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        futs = {ex.submit(_compile, s, e, objdir): s for s, e in SOURCES.items()}
        objs = [f.result() for f in futs]
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *sorted(objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    pobj = _compile("ts_probe.hip", [], objdir)
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", PROBE_PATH + ".tmp", pobj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(PROBE_PATH + ".tmp", PROBE_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {PROBE_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
