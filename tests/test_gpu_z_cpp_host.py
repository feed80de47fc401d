"""GPU: a C++ host over the C ABI alone (tests/c_abi/ffn_decode.cpp, built by __graft_entry__.build()): host
packing to 4352-byte tiles, device repack and hm_ffn_forward at M = 1, 3, 16 and 48, checked in the program
against a float64 evaluation of the same weights."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "ffn_decode")


def test_cpp_host_ffn_forward():
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build() first"
    print("running", BIN, flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "PASS" in r.stdout, (r.returncode, r.stdout, r.stderr)
