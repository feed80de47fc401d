"""GPU: seeded random shapes through the launch planners, against the float64 oracle on every row.

The hand-picked cases elsewhere pin each planner rule at the shapes it was written for. These draw the shape (K, N,
group, dtype, rows, a K prefix, a column or channel range) from a fixed seed, so rule boundaries that no hand-picked
case sits on are crossed too: one-row launches (with the K split past 256 K tiles), the few-row modes at 2..8 rows,
the several-row kernel at 9..16 rows with its cost-model launch shapes and K splits, and the GEMM's tile
configurations and K splits above 16 rows; for whole layers also the layer-stack block against the separate
operators, bit for bit. The case list is fixed at import (the same ids every run)."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu

MAX_WEIGHTS = 8 << 20  # logical weights per matrix, which keeps the float64 oracle to about a second per case


def _rows(rng):
    u = rng.random()
    if u < 0.25:
        return 1
    if u < 0.5:
        return int(rng.integers(2, 9))
    if u < 0.65:
        return int(rng.integers(9, 17))
    return int(rng.integers(17, 700))


def _linear_cases(count=96, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        group = int(rng.choice([32, 64, 128]))
        dtype = str(rng.choice(["fp16", "bf16"]))
        m = _rows(rng)
        if m <= 16 and rng.random() < 0.2:
            kt = int(rng.integers(200, 321))  # long K, narrow: the one-row K split past 256 K tiles
        else:
            kt = int(rng.integers(1, 49))
        k_used = kt if rng.random() < 0.8 else int(rng.integers(1, kt + 1))  # a prefix of the matrix's K
        unit = 16 if m <= 16 else 128  # the GEMM path takes whole 128-column blocks
        max_cols = max(unit, min(6144, MAX_WEIGHTS // (kt * 128)))
        n = unit * int(rng.integers(1, max_cols // unit + 1))
        col = 16 * int(rng.integers(1, 9)) if rng.random() < 0.4 else 0
        extra = 16 * int(rng.integers(0, 3))
        cases.append(pytest.param(m, kt * 128, k_used * 128, n, col, col + n + extra, group, dtype,
                                  id=f"{i}-m{m}-k{k_used * 128}of{kt * 128}-n{n}@{col}-g{group}-{dtype}"))
    return cases


def _ffn_cases(count=32, seed=20261203):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        group = int(rng.choice([32, 64, 128]))
        dtype = str(rng.choice(["fp16", "bf16"]))
        m = _rows(rng)
        hidden = 128 * int(rng.integers(1, 26))
        inter = 128 * int(rng.integers(1, min(49, (6 << 20) // (hidden * 128)) + 1))
        channels = None
        if rng.random() < 0.3 and inter > 128:
            b = 128 * int(rng.integers(0, inter // 128))
            e = b + 128 * int(rng.integers(1, (inter - b) // 128 + 1))
            channels = (b, e)
        tag = "all" if channels is None else f"{channels[0]}-{channels[1]}"
        cases.append(pytest.param(m, hidden, inter, channels, group, dtype, id=f"{i}-m{m}-h{hidden}-i{inter}-ch{tag}-g{group}-{dtype}"))
    return cases


@pytest.mark.parametrize("m,k,k_used,n,col,n_total,group,dtype", _linear_cases())
def test_linear_random_shape(oracle, hm, device, m, k, k_used, n, col, n_total, group, dtype):
    rng = np.random.default_rng([m, k, n, col, group])
    w_np = oracle.random_weights(rng, k, n_total, group, dtype)
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, dtype, device), group, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, k_used, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, w, k=k_used, n=n, col_begin=col)
    y2 = torch.empty_like(y)
    hm.packed_linear(y2, x, w, k=k_used, n=n, col_begin=col)
    torch.cuda.synchronize()
    ref = x64 @ oracle.weights_f64(*w_np, group, dtype)[:k_used, col:col + n]
    assert_close(oracle, host_f64(y), ref, dtype, f"linear M={m} K={k_used} of {k} cols [{col}, {col + n}) of {n_total} g={group}")
    assert torch.equal(y, y2), "a repeated call gives other bits"
    w.close()


@pytest.mark.parametrize("m,hidden,inter,channels,group,dtype", _ffn_cases())
def test_ffn_random_shape(oracle, hm, device, m, hidden, inter, channels, group, dtype):
    rng = np.random.default_rng([m, hidden, inter, group])
    mats = [oracle.random_weights(rng, k, n, group, dtype) for k, n in ((hidden, inter), (hidden, inter), (inter, hidden))]
    layer = hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in mats), group, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, hidden, dtype, device)
    y = layer.forward(x, channels=channels)
    torch.cuda.synchronize()
    b, e = (0, inter) if channels is None else channels
    wg, wu, wd = (oracle.weights_f64(*w, group, dtype) for w in mats)
    act = oracle.silu(x64 @ wg[:, b:e]) * (x64 @ wu[:, b:e])
    act = oracle.round_to(act.astype(np.float32), dtype).astype(np.float64)
    assert_close(oracle, host_f64(y), act @ wd[b:e], dtype, f"FFN M={m} H={hidden} I={inter} channels [{b}, {e}) g={group}")
    if channels is None:
        # the layer-stack block, x += FFN(RMSNorm(x) * w) in place: the same bits as rmsnorm, forward and residual_add2
        w = torch.from_numpy(rng.uniform(0.5, 1.5, hidden).astype(np.float32)).to(device).to(TORCH[dtype])
        ref = x.clone()
        normed = torch.empty_like(x)
        hm.rmsnorm(normed, ref, w, 1e-5)
        hm.residual_add2(ref, layer.forward(normed))
        got = x.clone()
        layer.block_forward(got, w, 1e-5)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), "block forward differs from the separate operators"
    layer.close()
