"""The C++ host side (include/turboshimmy.hpp) on the GPU: tests/cpp/test_int4_parity.cpp runs
the reference's INT4 parity tests (src/backend/bindless/test_int4_parity.rs:306-585) and
prefill / decode attention against the CPU oracle through the C++ KVCache, in one process.
Built by tests/cpp/Makefile (part of __graft_entry__.build())."""
import os
import subprocess

import pytest

from .gpu_util import say

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "_build", "test_int4_parity")


@pytest.mark.gpu
def test_cpp_host_side_parity():
    say("C++ host side: tests/cpp/test_int4_parity")
    assert os.path.exists(BIN), f"{BIN} is missing: build it with make -C tests/cpp"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, f"C++ parity tests failed:\n{r.stdout}\n{r.stderr}"
    assert r.stdout.count("PASS ") == 6
