"""GPU: hm_linear_split runs the split a config entry describes (M, N, K, and the GEMV's column shares) with every
share on the GPU. Row and column shares give the bits of the unsplit launch (no launch here splits K differently);
the K split equals hm_linear_k_split and the oracle's round(round(x0 W0) + round(x1 W1))."""

import numpy as np
import pytest
import torch

from gpu_util import assert_close, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gate(oracle, hm, device):
    w = oracle.random_weights(np.random.default_rng(1), 4096, 14336, 128, "bf16")
    return w, hm.RepackedMatrix.from_logical(*logical_to_device(w, "bf16", device), 128, dtype=torch.bfloat16)


def _run(hm, out, x, value, w0, w1=None):
    hm.hetero.hetero_linear(out, x, value, w0, w1)
    torch.cuda.synchronize()
    return out


def test_row_and_column_splits_equal_unsplit(oracle, hm, device, gate):
    w, rw = gate
    het = hm.hetero
    cm = het.ConfigMap()
    cm.add_gemm(2048, 4096, 14336, "gate", 512, 4096, 14336)    # M split: rows [0, 1536) and [1536, 2048)
    cm.add_gemm(1024, 4096, 14336, "gate", 1024, 4096, 7168)    # N split: columns [7168, 14336) then [0, 7168)
    cm.add_gemv(4096, 14336, "gate", npuN=4096, cpuN=1024)      # GEMV column shares
    cm.add_gemv(4096, 14336, "up", npuN=4096, cpuN=1000)        # cpuN not a multiple of 64: the GPU takes those columns
    rng = np.random.default_rng(2)
    wf = oracle.weights_f64(*w, 128, "bf16")
    for m, layer in ((2048, "gate"), (1024, "gate"), (1, "gate"), (1, "up")):
        value = cm.find(m, 4096, 14336, layer)
        assert value is not None
        x64, x = make_x(oracle, rng, m, 4096, "bf16", device)
        split = _run(hm, torch.full((m, 14336), float("nan"), dtype=torch.bfloat16, device=device), x, value, rw)
        whole = _run(hm, torch.empty((m, 14336), dtype=torch.bfloat16, device=device), x, None, rw)
        print(f"{layer} M={m}: split_type {value.split_type}, equal to the unsplit launch: {torch.equal(split, whole)}", flush=True)
        assert torch.equal(split, whole), (m, layer, value)
        sel = np.arange(m) if m <= 64 else np.sort(rng.choice(m, 48, replace=False))
        assert_close(oracle, host_f64(split)[sel], x64[sel] @ wf, "bf16", f"split {value.split_type} M={m}")


@pytest.mark.parametrize("m", [1, 3, 64])
def test_k_split_entry(oracle, hm, device, m):
    rng = np.random.default_rng(3)
    k0, k1, n = 7168, 7168, 4096  # a down projection split at K0 = 7168
    w0 = oracle.random_weights(rng, k0, n, 128, "bf16")
    w1 = oracle.random_weights(rng, k1, n, 128, "bf16")
    r0 = hm.RepackedMatrix.from_logical(*logical_to_device(w0, "bf16", device), 128, dtype=torch.bfloat16)
    r1 = hm.RepackedMatrix.from_logical(*logical_to_device(w1, "bf16", device), 128, dtype=torch.bfloat16)
    cm = hm.hetero.ConfigMap()
    cm.add_gemm(m, k0 + k1, n, "down", m, k0, n)
    value = cm.find(m, k0 + k1, n, "down")
    assert value.split_type == k0
    x64, x = make_x(oracle, rng, m, k0 + k1, "bf16", device)
    y = _run(hm, torch.empty((m, n), dtype=torch.bfloat16, device=device), x, value, r0, r1)
    ref = torch.empty_like(y)
    hm.packed_linear_k_split(ref, x, r0, r1)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    a = oracle.round_to((x64[:, :k0] @ oracle.weights_f64(*w0, 128, "bf16")).astype(np.float32), "bf16")
    b = oracle.round_to((x64[:, k0:] @ oracle.weights_f64(*w1, 128, "bf16")).astype(np.float32), "bf16")
    assert_close(oracle, host_f64(y), a.astype(np.float64) + b, "bf16", f"K split entry M={m}")
    with pytest.raises(ValueError):  # a K split without its second matrix
        hm.hetero.hetero_linear(torch.empty((m, n), dtype=torch.bfloat16, device=device), x, value, r0, None, k=k0 + k1)
