"""GPU: seeded random shapes through the launch planners, against the float64 oracle on every row.

The hand-picked cases elsewhere pin each planner rule at the shapes it was written for. These draw the shape (K, N,
group, dtype, rows, a K prefix, a column or channel range) from a fixed seed, so rule boundaries that no hand-picked
case sits on are crossed too: one-row launches (with the K split past 256 K tiles), the few-row modes at 2..8 rows,
the several-row kernel at 9..16 rows with its cost-model launch shapes and K splits, and the GEMM's tile
configurations and K splits above 16 rows; for whole layers also the layer-stack block against the separate
operators, bit for bit; the reference's fused gate_up tensor over channel ranges; and the K-split pair over two
matrices. The case lists are fixed at import (the same ids every run)."""

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


def _gate_up_cases(count=24, seed=20261204):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        dtype = str(rng.choice(["fp16", "bf16"]))
        layout = str(rng.choice(["interleaved", "blocked"]))
        m = _rows(rng)
        hidden = 128 * int(rng.integers(1, 17))
        stored = 64 * int(rng.integers(1, 65))
        unit = 16 if m <= 16 else 64  # the fused GEMM takes whole 64-channel blocks
        b = unit * int(rng.integers(0, stored // unit)) if rng.random() < 0.4 else 0
        e = b + unit * int(rng.integers(1, (stored - b) // unit + 1)) if rng.random() < 0.5 else stored
        cases.append(pytest.param(m, hidden, stored, (b, e), layout, dtype, id=f"{i}-m{m}-h{hidden}-s{stored}-ch{b}-{e}-{layout}-{dtype}"))
    return cases


@pytest.mark.parametrize("m,hidden,stored,channels,layout,dtype", _gate_up_cases())
def test_gate_up_tensor_random_shape(oracle, hm, device, m, hidden, stored, channels, layout, dtype):
    # The reference's fused gate_up tensor (4352-byte tiles, bf16 scales, group 128) through the SwiGLU projection
    # over a channel range; within tolerance of float64, and where the range falls on 128-channel blocks of a layer
    # whose stored channels do, bit-equal to the layer's gate_up from separate gate and up matrices.
    rng = np.random.default_rng([m, hidden, stored, channels[0], channels[1]])
    gate = oracle.random_weights(rng, hidden, stored, 128, "bf16")
    up = oracle.random_weights(rng, hidden, stored, 128, "bf16")
    gu = torch.from_numpy(oracle.pack_tiles(*oracle.join_gate_up(gate, up, layout))).to(device)
    w = hm.RepackedMatrix.from_gate_up_tiles(gu, hidden, stored, layout=layout, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, hidden, dtype, device)
    b, e = channels
    act = torch.empty((m, e - b), dtype=TORCH[dtype], device=device)
    hm.packed_linear_swiglu(act, x, w, channels=channels)
    torch.cuda.synchronize()
    # the tiles' bf16 scales become fp16 in an fp16 projection: the oracle takes the same rounded scales
    wg, wu = (oracle.weights_f64(q, oracle.to_bits(oracle.bf16_bits_to_f32(s), dtype), z, 128, dtype) for q, s, z in (gate, up))
    ref = oracle.silu(x64 @ wg[:, b:e]) * (x64 @ wu[:, b:e])
    assert_close(oracle, host_f64(act), ref, dtype, f"gate_up tensor ({layout}) M={m} H={hidden} channels [{b}, {e}) of {stored}")
    if stored % 128 == 0 and b % 128 == 0 and e % 128 == 0:
        down = torch.from_numpy(oracle.pack_tiles(*oracle.random_weights(rng, stored, hidden, 128, "bf16"))).to(device)
        tiles = [torch.from_numpy(oracle.pack_tiles(*t)).to(device) for t in (gate, up)]
        layer = hm.FfnLayer.from_tiles(*tiles, down, hidden, stored, dtype=TORCH[dtype])
        ref_bits = layer.gate_up(x, channels=channels)
        torch.cuda.synchronize()
        assert torch.equal(act, ref_bits), "the gate_up tensor route differs from the two-matrix route"
        layer.close()
    w.close()


def _k_split_cases(count=24, seed=20261205):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        group = int(rng.choice([32, 64, 128]))
        dtype = str(rng.choice(["fp16", "bf16"]))
        m = _rows(rng)
        k0 = 128 * int(rng.integers(1, 33))
        k1 = k0 if rng.random() < 0.2 else 128 * int(rng.integers(1, 33))
        unit = 16 if m <= 16 else 128
        n = unit * int(rng.integers(1, max(2, MAX_WEIGHTS // (max(k0, k1) * unit)) // 2 + 1))
        cases.append(pytest.param(m, k0, k1, n, group, dtype, id=f"{i}-m{m}-k{k0}+{k1}-n{n}-g{group}-{dtype}"))
    return cases


@pytest.mark.parametrize("m,k0,k1,n,group,dtype", _k_split_cases())
def test_k_split_pair_random_shape(oracle, hm, device, m, k0, k1, n, group, dtype):
    # A K split over two matrices (hetero_matmul_out_gem{v,m}_packed_K with both shares on the GPU): within tolerance
    # of round(round(a) + round(b)) in float64; from two rows, and at one row when the shares run as two launches,
    # the bits of the two projections added by torch.
    rng = np.random.default_rng([m, k0, k1, n, group])
    w_np = [oracle.random_weights(rng, k, n, group, dtype) for k in (k0, k1)]
    w0, w1 = (hm.RepackedMatrix.from_logical(*logical_to_device(t, dtype, device), group, dtype=TORCH[dtype]) for t in w_np)
    x64, x = make_x(oracle, rng, m, k0 + k1, dtype, device)
    y = torch.full((m, n), float("nan"), dtype=TORCH[dtype], device=device)
    hm.packed_linear_k_split(y, x, w0, w1)
    y0 = hm.packed_linear(torch.empty((m, n), dtype=TORCH[dtype], device=device), x[:, :k0], w0)
    y1 = hm.packed_linear(torch.empty((m, n), dtype=TORCH[dtype], device=device), x[:, k0:], w1)
    torch.cuda.synchronize()
    a, b = (oracle.round_to((xs @ oracle.weights_f64(*t, group, dtype)).astype(np.float32), dtype).astype(np.float64)
            for xs, t in ((x64[:, :k0], w_np[0]), (x64[:, k0:], w_np[1])))
    assert_close(oracle, host_f64(y), a + b, dtype, f"K split {k0}+{k1} M={m} n={n} g={group}")
    if m > 1:
        assert torch.equal(y, y0 + y1), "the second share's accumulating epilogue differs from a separate add"
    w0.close()
    w1.close()
