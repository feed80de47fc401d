"""GPU: decode GEMVs at several rows against the float64 oracle, through the C ABI, on shapes chosen to reach
the multi-row launch-shape rule's corners: narrow outputs split along K (up to 16 splits, several waves per strip
group reducing through LDS), wide outputs with one wave per strip group, odd row counts (rows padded to a
multiple of 4 in the staged chunk), the fused SwiGLU, and zero points up to 16 (the largest a GPTQ checkpoint
gives after adding its one back), which the multi-row kernel takes off with the exact operand -(bias + z).
Two to four rows run the one-row math with one row per lane group (their own tests below)."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("m", [1, 3, 16, 40])
def test_zero_point_sixteen(oracle, hm, device, dtype, m):
    rng = np.random.default_rng(700 + m)
    k, n, g = 1024, 512, 128
    w_np = oracle.random_weights(rng, k, n, g, dtype, z_lo=12, z_hi=17)
    assert w_np[2].max() == 16
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, dtype, device), g, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, g, dtype), dtype, f"zero 16 M={m}")


@pytest.mark.parametrize("m", [2, 6, 11, 16])
@pytest.mark.parametrize("k,n,g,dtype", [
    (8192, 256, 128, "fp16"),   # 8 strip pairs: many K splits, several waves per group
    (4096, 1024, 64, "bf16"),   # narrow, groups of 64 (shallower ring)
    (1024, 8192, 128, "fp16"),  # wide: one wave per strip group, no split
    (2048, 2048, 32, "fp16"),   # groups of 32
])
def test_multirow_launch_shapes(oracle, hm, device, m, k, n, g, dtype):
    rng = np.random.default_rng(800 + m + k // 128 + n // 16 + g)
    w_np = oracle.random_weights(rng, k, n, g, dtype)
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, dtype, device), g, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, g, dtype), dtype, f"linear M={m} [{k}x{n}] g={g} {dtype}")


@pytest.mark.parametrize("m", [3, 8, 13])
def test_multirow_fused_gate_up(oracle, hm, device, m):
    # A small FFN's gate_up at several rows: SwiGLU of the two strips of each pair, written from the first wave of
    # the strip group (or by sum_splits where the rule splits K), against the oracle's single-rounding SwiGLU.
    rng = np.random.default_rng(900 + m)
    hidden, inter, g, dtype = 2048, 3072, 128, "fp16"
    gate_np = oracle.random_weights(rng, hidden, inter, g, dtype)
    up_np = oracle.random_weights(rng, hidden, inter, g, dtype)
    down_np = oracle.random_weights(rng, inter, hidden, g, dtype)
    ffn = hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in (gate_np, up_np, down_np)), g, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, hidden, dtype, device)
    act = torch.empty((m, inter), dtype=TORCH[dtype], device=device)
    ffn.gate_up(x, act)
    torch.cuda.synchronize()
    gate = x64 @ oracle.weights_f64(*gate_np, g, dtype)
    up = x64 @ oracle.weights_f64(*up_np, g, dtype)
    ref = oracle.silu(gate) * up
    assert_close(oracle, host_f64(act), ref, dtype, f"gate_up M={m}")


@pytest.mark.parametrize("m", [2, 5, 8, 16])
@pytest.mark.parametrize("hidden,inter,group,dtype", [
    (4096, 14336, 128, "fp16"),   # Llama-3-8B: the down GEMV splits K from 5 rows on
    (5120, 13824, 64, "bf16"),    # Qwen2.5-14B
    (2048, 8192, 128, "fp16"),    # Llama-3.2-1B
])
def test_forward_equals_separate_calls(oracle, hm, device, m, hidden, inter, group, dtype):
    # hm_ffn_forward at 2..16 rows against hm_ffn_gate_up then hm_ffn_down on the caller's act: the same bits,
    # including the down GEMV's K-split partials and their sum, on two calls in a row over one workspace.
    rng = np.random.default_rng(1000 + m + hidden)
    ws = [oracle.random_weights(rng, k, n, group, dtype) for k, n in ((hidden, inter), (hidden, inter), (inter, hidden))]
    ffn = hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in ws), group, dtype=TORCH[dtype])
    print(f"forward M={m} [{hidden} x {inter}] g={group} {dtype}", flush=True)
    for rep in range(2):
        _, x = make_x(oracle, rng, m, hidden, dtype, device)
        y = ffn.forward(x)
        ref = ffn.down(ffn.gate_up(x))
        torch.cuda.synchronize()
        assert torch.equal(y, ref), (m, hidden, dtype, rep)


@pytest.mark.parametrize("m", [2, 3, 4, 5, 7, 8])
@pytest.mark.parametrize("k,n,g,dtype", [
    (14336, 512, 128, "fp16"),  # the Llama-3-8B down's K: 8 waves of 14 K tiles per strip, whose rows' 1 KiB transfers
                                # overlap; up to 5 rows unsplit (150 KiB of LDS at 5)
    (2688, 768, 64, "bf16"),    # 21 K tiles: each staged row rounded up to whole transfers; groups of 64
    (3072, 1024, 32, "fp16"),   # groups of 32 (the ring sized by the kernel)
    (28672, 128, 128, "fp16"),  # 224 K tiles: at 3 and 4 rows the staged rows exceed LDS and K splits in two
    (4096, 2048, 128, "bf16"),  # bf16 at group 128, five to eight rows on two rows per lane group
])
def test_few_rows_shapes(oracle, hm, device, m, k, n, g, dtype):
    # Two to four rows (any group) and, where the rows fit LDS whole, five to eight (groups of 128): x rows staged one
    # after another by DMA, group sums per row, lane group h of the MFMA output carrying rows R h .. R h + R - 1
    # (R = 1, 2); every row against float64. The other shapes at five to eight rows take the several-row kernel.
    rng = np.random.default_rng(1100 + m + k // 128 + g)
    w_np = oracle.random_weights(rng, k, n, g, dtype)
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, dtype, device), g, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    print(f"few rows M={m} [{k}x{n}] g={g} {dtype}", flush=True)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, g, dtype), dtype, f"few rows M={m} [{k}x{n}] g={g} {dtype}")


@pytest.mark.parametrize("m", [2, 4])
@pytest.mark.parametrize("group,dtype", [(32, "fp16"), (64, "bf16"), (128, "bf16")])
def test_few_rows_fused_gate_up_groups(oracle, hm, device, m, group, dtype):
    # The few-row fused gate_up (SiLU(gate) * up from the lane's two strips, one rounding) at groups of 32 / 64 / 128 and
    # both activation types, every output against the oracle's single-rounding SwiGLU.
    rng = np.random.default_rng(1300 + m + group)
    hidden, inter = 2048, 1536
    ws = [oracle.random_weights(rng, kk, nn, group, dtype) for kk, nn in ((hidden, inter), (hidden, inter), (inter, hidden))]
    ffn = hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in ws), group, dtype=TORCH[dtype])
    x64, x = make_x(oracle, rng, m, hidden, dtype, device)
    act = torch.empty((m, inter), dtype=TORCH[dtype], device=device)
    ffn.gate_up(x, act)
    torch.cuda.synchronize()
    ref = oracle.silu(x64 @ oracle.weights_f64(*ws[0], group, dtype)) * (x64 @ oracle.weights_f64(*ws[1], group, dtype))
    assert_close(oracle, host_f64(act), ref, dtype, f"few-row gate_up M={m} g={group} {dtype}")


@pytest.mark.parametrize("m", [12, 16])
def test_multirow_long_k_split_fallback(oracle, hm, device, m):
    # A long K at 12 or 16 rows (a Llama-3-70B down projection, K = 28672, N = 8192): the staged chunk needs at least
    # six K splits, which the planner's bound on split partials does not allow. The plan takes the fewest splits that
    # fit LDS (six), so the workspace stays a few MB (224 one-tile splits would need 84-112 MB of partials).
    rng = np.random.default_rng(900 + m)
    k, n, g, dtype = 28672, 8192, 128, "fp16"
    w_np = oracle.random_weights(rng, k, n, g, dtype)
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, dtype, device), g, dtype=TORCH[dtype])
    ws = w.workspace_bytes(m)
    print(f"workspace at M={m}: {ws} bytes")
    assert ws <= 6 * m * n * 4 + (1 << 20)
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    cols = np.r_[0:64, 4000:4064, n - 64:n]  # three strips' worth of columns, against float64 on those columns
    wf = oracle.dequantize(w_np[0][:, cols], oracle.from_bits(w_np[1][:, cols], dtype), w_np[2][:, cols], g)
    assert_close(oracle, host_f64(y)[:, cols], x64 @ wf, dtype, f"long K M={m}")
