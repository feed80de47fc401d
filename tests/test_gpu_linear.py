"""GPU: one projection y = x W (decode GEMV for M <= 16, MFMA GEMM above) against the float64 oracle, through
the C ABI. Covers both dtypes, groups 32/64/128, ragged M, prefixes (leading blocks), start columns and the
split-K path."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, dev, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu


def _matrix(oracle, hm, rng, k, n, group, dtype, device):
    w_np = oracle.random_weights(rng, k, n, group, dtype)
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, dtype, device), group, dtype=TORCH[dtype])
    return w_np, w


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 9, 16, 17, 37, 128, 300])
def test_linear_vs_oracle(oracle, hm, device, dtype, m):
    rng = np.random.default_rng(100 + m)
    k, n, g = 2048, 1024, 128
    w_np, w = _matrix(oracle, hm, rng, k, n, g, dtype, device)
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    ref = x64 @ oracle.weights_f64(*w_np, g, dtype)
    assert_close(oracle, host_f64(y), ref, dtype, f"linear M={m} [{k}x{n}] g={g}")


@pytest.mark.parametrize("m", [1, 16, 200])
def test_linear_tiny_scales(oracle, hm, device, m):
    # fp16 scales below 2^-10 (and subnormal ones): the GEMM's odd pairs multiply by s / 16, which then loses
    # low bits; the result must stay within the tolerance.
    rng = np.random.default_rng(150 + m)
    k, n, g = 1024, 512, 128
    w_np = oracle.random_weights(rng, k, n, g, "fp16", 1e-6, 9e-4)
    w = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, "fp16", device), g, dtype=torch.float16)
    x64, x = make_x(oracle, rng, m, k, "fp16", device)
    y = torch.empty((m, n), dtype=torch.float16, device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    ref = x64 @ oracle.weights_f64(*w_np, g, "fp16")
    assert_close(oracle, host_f64(y), ref, "fp16", f"tiny scales M={m}")


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_linear_small_groups(oracle, hm, device, group, m):
    rng = np.random.default_rng(200 + group + m)
    k, n, dtype = 1024, 512, "fp16"
    w_np, w = _matrix(oracle, hm, rng, k, n, group, dtype, device)
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=torch.float16, device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, group, dtype), dtype, f"linear g={group} M={m}")


@pytest.mark.parametrize("m", [1, 3, 16, 128])
def test_linear_prefix_and_start_column(oracle, hm, device, m):
    # leading k x n block of a larger matrix, and columns [col, col + n)
    rng = np.random.default_rng(300 + m)
    K, N, dtype = 2048, 1024, "bf16"
    w_np, w = _matrix(oracle, hm, rng, K, N, 128, dtype, device)
    wf = oracle.weights_f64(*w_np, 128, dtype)
    for k, n, col in [(1024, 512, 0), (2048, 256, 512), (512, 128, 896)]:
        x64, x = make_x(oracle, rng, m, k, dtype, device)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        hm.packed_linear(y, x, w, k=k, n=n, col_begin=col)
        torch.cuda.synchronize()
        assert_close(oracle, host_f64(y), x64 @ wf[:k, col:col + n], dtype, f"prefix k={k} n={n} col={col} M={m}")


@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("m", [2, 16])
def test_linear_odd_strip_count(oracle, hm, device, group, m):
    # 5 strips of 16 columns: M > 1 cannot pair strips per wave, so one strip per wave; 3 K tiles leave
    # waves without tiles.
    rng = np.random.default_rng(600 + group + m)
    k, n, dtype = 384, 80, "bf16"
    w_np, w = _matrix(oracle, hm, rng, k, n, group, dtype, device)
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, group, dtype), dtype, f"odd strips g={group} M={m}")


@pytest.mark.parametrize("k1", [128, 256])
def test_linear_waves_without_tiles(oracle, hm, device, k1):
    # A K-split pair at one row runs both shares in one GEMV launch with the longer share's wave split: 8 waves per
    # strip for the 64 K tiles of share 0, so the 1 or 2 K tiles of share 1 leave waves of its split with no tile.
    # Their steps must not leak anything (they read LDS that no wave of their range staged).
    rng = np.random.default_rng(700 + k1)
    k0, n, dtype = 8192, 64, "fp16"
    w0_np, w0 = _matrix(oracle, hm, rng, k0, n, 128, dtype, device)
    w1_np, w1 = _matrix(oracle, hm, rng, k1, n, 128, dtype, device)
    x64, x = make_x(oracle, rng, 1, k0 + k1, dtype, device)
    y = torch.empty((1, n), dtype=torch.float16, device=device)
    hm.packed_linear_k_split(y, x, w0, w1)
    torch.cuda.synchronize()
    a = oracle.round_to((x64[:, :k0] @ oracle.weights_f64(*w0_np, 128, dtype)).astype(np.float32), dtype)
    b = oracle.round_to((x64[:, k0:] @ oracle.weights_f64(*w1_np, 128, dtype)).astype(np.float32), dtype)
    assert_close(oracle, host_f64(y), a.astype(np.float64) + b, dtype, f"idle waves k1={k1}")


def test_linear_split_k_path(oracle, hm, device):
    # M = 16 with K = 14336 does not fit the activation stage in LDS: the GEMV splits K and sums partials.
    rng = np.random.default_rng(400)
    k, n, dtype = 14336, 512, "fp16"
    w_np, w = _matrix(oracle, hm, rng, k, n, 128, dtype, device)
    assert w.workspace_bytes(16) > 0
    x64, x = make_x(oracle, rng, 16, k, dtype, device)
    y = torch.empty((16, n), dtype=torch.float16, device=device)
    hm.packed_linear(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, 128, dtype), dtype, "split-K M=16 K=14336")


def test_linear_strided_rows(oracle, hm, device):
    # x and y as row views of wider buffers (leading dimensions > width)
    rng = np.random.default_rng(500)
    k, n, dtype = 1024, 256, "fp16"
    w_np, w = _matrix(oracle, hm, rng, k, n, 128, dtype, device)
    for m in (1, 8, 40):
        x64, xw = make_x(oracle, rng, m, k + 64, dtype, device)
        yw = torch.zeros((m, n + 32), dtype=torch.float16, device=device)
        hm.packed_linear(yw[:, :n], xw[:, :k], w)
        torch.cuda.synchronize()
        assert_close(oracle, host_f64(yw[:, :n]), x64[:, :k] @ oracle.weights_f64(*w_np, 128, dtype), dtype, f"strided M={m}")
        assert torch.all(yw[:, n:] == 0)


def test_reference_tiles_decode_path(oracle, hm, device):
    # The drop-in route: bf16 weights from reference 4352-byte tiles, M = 1 (hipkernels::w4a16_gemv_fused_packed).
    rng = np.random.default_rng(600)
    k, n = 4096, 1024
    w_np = oracle.random_weights(rng, k, n, 128, "bf16", 0.002, 0.02, 6, 10)
    w = hm.RepackedMatrix.from_tiles(dev(oracle.pack_tiles(*w_np), device), k, n, dtype=torch.bfloat16)
    x64, x = make_x(oracle, rng, 1, k, "bf16", device, 0.5)
    y = torch.empty((1, n), dtype=torch.bfloat16, device=device)
    hm.gemv_w4a16(y, x, w)
    torch.cuda.synchronize()
    assert_close(oracle, host_f64(y), x64 @ oracle.weights_f64(*w_np, 128, "bf16"), "bf16", "tiles gemv")


def test_constant_input_exact(oracle, hm, device):
    # x = 1/16, q = 9, z = 8, s = 1/16, K = 2048 gives exactly 8 (docs/progress.md:457-460), decode and GEMM.
    k, n = 2048, 64
    q = torch.full((k, n), 9, dtype=torch.uint8, device=device)
    z = torch.full((k // 128, n), 8, dtype=torch.uint8, device=device)
    for dt in (torch.float16, torch.bfloat16):
        s = torch.full((k // 128, n), 1 / 16, dtype=dt, device=device)
        w = hm.RepackedMatrix.from_logical(q, s, z, 128, dtype=dt)
        for m in (1, 4, 300):
            x = torch.full((m, k), 1 / 16, dtype=dt, device=device)
            y = torch.empty((m, n), dtype=dt, device=device) if n % 128 == 0 or m <= 16 else None
            if y is None:
                continue
            hm.packed_linear(y, x, w)
            torch.cuda.synchronize()
            assert torch.all(y.float() == 8.0), (dt, m)


@pytest.mark.parametrize("m", [1, 8, 37, 512, 2048, 4096])
def test_concat_qkv_equals_separate(oracle, hm, device, m):
    # The Q, K and V projections of a Llama-3-8B attention block (grouped K/V: 4096, 1024 and 1024 columns) as
    # one matrix and one launch. Bit for bit against three launches at one row and where no GEMM launch splits K
    # (M = 4096 here: an output column's sum then does not depend on the other columns); within tolerance at
    # 2..16 rows, where the GEMV's K split follows the matrix width, and at M = 37..2048, where the narrow K/V
    # launches (small grids) split K and the wide one does not. The concatenated planes decode to the parts'
    # logical tensors side by side.
    rng = np.random.default_rng(120)
    k, g, dtype = 4096, 128, "fp16"
    parts = [_matrix(oracle, hm, rng, k, n, g, dtype, device) for n in (4096, 1024, 1024)]
    qkv = hm.RepackedMatrix.concat([w for _, w in parts])
    assert (qkv.k, qkv.n, qkv.group) == (k, 6144, g)
    q, s, z = qkv.to_logical()
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), np.concatenate([w_np[0] for w_np, _ in parts], axis=1))
    assert np.array_equal(z.cpu().numpy(), np.concatenate([w_np[2] for w_np, _ in parts], axis=1))
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, qkv.n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, qkv)
    sep = [hm.packed_linear(torch.empty((m, w.n), dtype=TORCH[dtype], device=device), x, w) for _, w in parts]
    torch.cuda.synchronize()
    ref = torch.cat(sep, dim=1)
    if m == 1 or m == 4096:
        assert torch.equal(y, ref)
    else:
        assert_close(oracle, host_f64(y), host_f64(ref), dtype, f"QKV one launch vs three M={m}")
    wf = np.concatenate([oracle.weights_f64(*w_np, g, dtype) for w_np, _ in parts], axis=1)
    sel = np.arange(m) if m <= 512 else np.sort(rng.choice(m, 64, replace=False))
    assert_close(oracle, host_f64(y)[sel], x64[sel] @ wf, dtype, f"QKV M={m}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("m", [1, 4, 16, 37, 512, 2048])
@pytest.mark.parametrize("k0,k1", [(2560, 1536), (1536, 2560), (2048, 2048)])
def test_linear_k_split_pair(oracle, hm, device, dtype, m, k0, k1):
    # A K-split pair (rows [0, k0) and [k0, k0 + k1) of a [4096, 1024] projection) with both shares on the GPU
    # (hetero_matmul_out_gem{v,m}_packed_K, GPU-only): the reference's sum of the two shares' rounded outputs
    # (out.add_(temp), here torch's add of two separate launches), and within tolerance of the oracle's
    # round(round(a) + round(b)). At one row both shares run in one launch with the longer share's wave split,
    # so their sums take the separate launches' order (and bits) when k0 == k1 and within rounding otherwise.
    # From 4 rows the second share adds into the output in the split sums (M = 4, 16; the GEMM at M = 37 and
    # 512 when its 20 K tiles split) or in the GEMM epilogue, bit for bit.
    rng = np.random.default_rng(140 + m + k0)
    n, g = 1024, 128
    w0_np, w0 = _matrix(oracle, hm, rng, k0, n, g, dtype, device)
    w1_np, w1 = _matrix(oracle, hm, rng, k1, n, g, dtype, device)
    x64, x = make_x(oracle, rng, m, k0 + k1, dtype, device)
    y = torch.full((m, n), float("nan"), dtype=TORCH[dtype], device=device)
    hm.packed_linear_k_split(y, x, w0, w1)
    y0 = hm.packed_linear(torch.empty((m, n), dtype=TORCH[dtype], device=device), x[:, :k0], w0)
    y1 = hm.packed_linear(torch.empty((m, n), dtype=TORCH[dtype], device=device), x[:, k0:], w1)
    torch.cuda.synchronize()
    if m == 1 and k0 != k1:
        assert_close(oracle, host_f64(y), host_f64(y0 + y1), dtype, f"K split pair in one launch {k0}+{k1}")
    else:
        assert torch.equal(y, y0 + y1)
    a = oracle.round_to((x64[:, :k0] @ oracle.weights_f64(*w0_np, g, dtype)).astype(np.float32), dtype).astype(np.float64)
    b = oracle.round_to((x64[:, k0:] @ oracle.weights_f64(*w1_np, g, dtype)).astype(np.float32), dtype).astype(np.float64)
    assert_close(oracle, host_f64(y), a + b, dtype, f"K split {k0}+{k1} M={m}")
    if m == 1:
        with pytest.raises(ValueError):
            hm.packed_linear_k_split(y, x, w0, w1, n=1040)
        with pytest.raises(ValueError):
            hm.packed_linear_k_split(y, x, w0, w1, k0=k0 - 64)


@pytest.mark.parametrize("m,k,n,col,g,dtype", [
    (17, 2048, 1024, 0, 128, "fp16"),     # 8 workgroups: K split in 2 (8 tiles each)
    (100, 4096, 512, 0, 64, "bf16"),      # group 64, 8 workgroups: K split in 4
    (130, 2560, 768, 0, 32, "fp16"),      # group 32, 18 workgroups: 20 K tiles split 10 + 10
    (257, 3072, 1280, 0, 64, "bf16"),     # 50 workgroups: 24 K tiles split in 3
    (300, 6144, 4096, 0, 128, "fp16"),    # 160 four-wave workgroups: split in 2 toward two per CU
    (300, 6144, 4096, 0, 128, "bf16"),
    (64, 1024, 128, 0, 128, "fp16"),      # 8 K tiles: too few to split
    (1000, 1024, 2048, 0, 128, "fp16"),   # 256 four-wave workgroups, 8 K tiles: no split
    (33, 2048, 384, 256, 128, "fp16"),    # a column range on the GEMM path, split in 2
    (9, 2048, 96, 512, 128, "bf16"),      # a column range on the GEMV path
])
def test_linear_planner_shapes(oracle, hm, device, m, k, n, col, g, dtype):
    # Launch plans across the GEMM's K-split rules (small grids toward 256 workgroups, 4-wave grids toward two
    # per CU, ragged splits, group 32 / 64, column ranges) against the oracle on every row.
    rng = np.random.default_rng(160 + m + k // 128)
    w_np, w = _matrix(oracle, hm, rng, k, col + n + 128, g, dtype, device)
    x64, x = make_x(oracle, rng, m, k, dtype, device)
    y = torch.empty((m, n), dtype=TORCH[dtype], device=device)
    hm.packed_linear(y, x, w, n=n, col_begin=col)
    torch.cuda.synchronize()
    ref = x64 @ oracle.weights_f64(*w_np, g, dtype)[:, col:col + n]
    assert_close(oracle, host_f64(y), ref, dtype, f"linear M={m} K={k} cols [{col}, {col + n}) g={g}")
