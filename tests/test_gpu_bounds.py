"""GPU: the kernels write nothing outside the caller's output block and workspace.

Every call gets an output view inside a larger allocation whose other rows and columns hold a sentinel, and a
workspace followed by guard bytes; after the call the sentinels and guards must be unchanged. Covers ragged M on
GEMM grids that split K and grids that do not (the epilogue drops rows past M through the buffer range check),
the decode GEMV, the K-split pair's accumulating epilogue and the FFN layer."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu

SENTINEL = 0x7E5A  # a finite value in both fp16 and bf16
GUARD = 0xA5
EXTRA_ROWS, EXTRA_COLS, GUARD_BYTES = 160, 48, 1 << 20


def _framed(m, n, dtype, device):
    """A [m + EXTRA_ROWS, n + EXTRA_COLS] sentinel frame and the [m, n] view (leading dimension n + EXTRA_COLS) the call writes."""
    big = torch.full((m + EXTRA_ROWS, n + EXTRA_COLS), SENTINEL, dtype=torch.int16, device=device).view(TORCH[dtype])
    return big, big[:m, :n]


def _frame_intact(big, m, n):
    bits = big.view(torch.int16)
    outside = torch.ones(bits.shape, dtype=torch.bool, device=bits.device)
    outside[:m, :n] = False
    return bool((bits[outside] == SENTINEL).all())


def _guarded_workspace(need, device):
    ws = torch.full((need + GUARD_BYTES + 256,), GUARD, dtype=torch.uint8, device=device)
    off = (-ws.data_ptr()) % 256
    return ws, off


def _guard_intact(ws, off, need):
    return bool((ws[off + need:] == GUARD).all())


def _weights(oracle, hm, device, k, n, group, dtype, seed):
    rng = np.random.default_rng(seed)
    w = oracle.random_weights(rng, k, n, group, dtype)
    return w, hm.RepackedMatrix.from_logical(*logical_to_device(w, dtype, device), group, dtype=TORCH[dtype])


# (k, n, m) and the launch each gets from the planner: 64 x 128 tiles with K split in 2, 2, 4 (m = 37, 100, 300 at
# n = 1024: 8, 16 and 40 workgroups); 64 x 128 tiles, 160 workgroups, no split (m = 600); 128 x 256 tiles, 256
# workgroups, no split (m = 1999); 128 x 128 tiles, 192 workgroups, no split (m = 300 at n = 8192); the decode
# GEMV (m = 5, 16). Every GEMM case has a last row tile that ends inside the tile.
CASES = [(2048, 1024, 37), (2048, 1024, 100), (4096, 1024, 300), (2048, 2048, 600), (2048, 4096, 1999), (2048, 8192, 300),
         (1024, 512, 5), (2048, 1024, 16)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("k,n,m", CASES)
def test_linear_writes_only_its_block(oracle, hm, device, dtype, k, n, m):
    w, rw = _weights(oracle, hm, device, k, n, 128, dtype, k + n + m)
    rng = np.random.default_rng(m)
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    big, y = _framed(m, n, dtype, device)
    lib = hm._lib.load()
    need = lib.hm_linear_workspace_bytes(rw._h, m, k, n)
    ws, off = _guarded_workspace(need, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"case k={k} n={n} m={m} {dtype} workspace={need}", flush=True)
    hm._lib.check(lib.hm_linear(rw._h, ctypes.c_void_p(y.data_ptr()), big.stride(0), ctypes.c_void_p(x.data_ptr()), x.stride(0), m, k, n,
                                0, ctypes.c_void_p(ws.data_ptr() + off), need, stream))
    torch.cuda.synchronize()
    assert _frame_intact(big, m, n), "a kernel wrote outside the [M, n] output block"
    assert _guard_intact(ws, off, need), "a kernel wrote past the workspace"
    sel = np.arange(m) if m <= 128 else np.sort(rng.choice(m, 64, replace=False))
    ref = x64[sel] @ oracle.weights_f64(*w, 128, dtype)
    assert_close(oracle, host_f64(y)[sel], ref, dtype, f"framed linear k={k} n={n} m={m}")


@pytest.mark.parametrize("m", [1, 7, 37, 300])
def test_k_split_pair_accumulate_writes_only_its_block(oracle, hm, device, m):
    dtype, k0, k1, n = "fp16", 1536, 2560, 1024
    w0, r0 = _weights(oracle, hm, device, k0, n, 128, dtype, 1)
    w1, r1 = _weights(oracle, hm, device, k1, n, 128, dtype, 2)
    rng = np.random.default_rng(100 + m)
    x64, x = make_x(oracle, rng, m, k0 + k1, dtype, device)
    big, y = _framed(m, n, dtype, device)
    lib = hm._lib.load()
    need = lib.hm_linear_k_split_workspace_bytes(r0._h, r1._h, m, k0, k1, n)
    ws, off = _guarded_workspace(need, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"case k-split m={m} workspace={need}", flush=True)
    hm._lib.check(lib.hm_linear_k_split(r0._h, r1._h, ctypes.c_void_p(y.data_ptr()), big.stride(0), ctypes.c_void_p(x.data_ptr()),
                                        x.stride(0), m, k0, k1, n, ctypes.c_void_p(ws.data_ptr() + off), need, stream))
    torch.cuda.synchronize()
    assert _frame_intact(big, m, n)
    assert _guard_intact(ws, off, need)
    ref = x64[:, :k0] @ oracle.weights_f64(*w0, 128, dtype)
    ref = oracle.round_to(ref.astype(np.float32), dtype) + oracle.round_to((x64[:, k0:] @ oracle.weights_f64(*w1, 128, dtype)).astype(np.float32), dtype)
    assert_close(oracle, host_f64(y), ref, dtype, f"framed k-split m={m}")


# (1000, 3584): the fused gate_up GEMM runs 8 row tiles of 128, the last one ragged.
@pytest.mark.parametrize("m,inter", [(1, 2816), (3, 2816), (37, 2816), (333, 2816), (1000, 3584)])
def test_ffn_writes_only_its_block(oracle, hm, device, m, inter):
    dtype, hidden, group = "bf16", 2048, 128
    rng = np.random.default_rng(7)
    ws_ = [oracle.random_weights(rng, hidden, inter, group, dtype), oracle.random_weights(rng, hidden, inter, group, dtype),
           oracle.random_weights(rng, inter, hidden, group, dtype)]
    layer = hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in ws_), group, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, hidden, dtype, device)
    big, y = _framed(m, hidden, dtype, device)
    lib = hm._lib.load()
    need = lib.hm_ffn_workspace_bytes(layer._h, m)
    ws, off = _guarded_workspace(need, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"case ffn m={m} workspace={need}", flush=True)
    hm._lib.check(lib.hm_ffn_forward(layer._h, ctypes.c_void_p(y.data_ptr()), big.stride(0), ctypes.c_void_p(x.data_ptr()), x.stride(0), m,
                                     0, inter, ctypes.c_void_p(ws.data_ptr() + off), need, stream))
    torch.cuda.synchronize()
    assert _frame_intact(big, m, hidden)
    assert _guard_intact(ws, off, need)
    ref, _ = oracle.ffn(x64, *ws_, group, dtype)
    assert_close(oracle, host_f64(y), ref, dtype, f"framed ffn m={m}")
