"""GPU: the layer-boundary operators beside the FFN (heteromega::residual_add2 with fp32 partials, residual_norm_bf16's
two-addend residual and norm) and the merged FFN's nonfinite scan on the device, against float32 emulations of the
same arithmetic (bit for bit), the float64 oracle (within tolerance) and the host scan."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, dev, host_bits, host_f64, make_x

pytestmark = pytest.mark.gpu


def _f32(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("g32,n32", [(False, True), (True, False), (True, True)])
def test_residual_add2_fp32_partials(oracle, hm, device, dtype, g32, n32):
    # x += y_g + y_n with either partial in fp32 (residual_add.cu:9-31, :61-72): partials added first, then the
    # residual, one rounding. The float32 emulation below is that arithmetic step by step, so the bits must agree.
    rng = np.random.default_rng(7 + 2 * g32 + n32)
    m, h = 5, 4096
    _, x = make_x(oracle, rng, m, h, dtype, device)
    yg = torch.from_numpy((rng.standard_normal((m, h)) * 0.7).astype(np.float32)).to(device)
    yn = torch.from_numpy((rng.standard_normal((m, h)) * 0.7).astype(np.float32)).to(device)
    if not g32:
        yg = yg.to(TORCH[dtype])
    if not n32:
        yn = yn.to(TORCH[dtype])
    want = oracle.to_bits(_f32(x) + (_f32(yg) + _f32(yn)), dtype)
    xr = x.clone()
    hm.residual_add2(xr, yg, yn)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(xr), want)
    with pytest.raises(ValueError):
        hm.residual_add2(x.clone(), yg if g32 else yn, None)  # fp32 partials come in pairs


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_residual_norm_two_addends(oracle, hm, device, dtype):
    # x = round((x + a) + b) (residual_norm.cu:45-49), then normed = RMSNorm(x) * w: the residual bit for bit against its
    # float32 emulation, the norm bit for bit against hm_rmsnorm of the updated x and within tolerance of float64.
    rng = np.random.default_rng(11)
    m, h = 17, 4096
    _, x = make_x(oracle, rng, m, h, dtype, device)
    _, a = make_x(oracle, rng, m, h, dtype, device, 0.3)
    _, b = make_x(oracle, rng, m, h, dtype, device, 0.3)
    w = (torch.rand((h,), device=device) + 0.5).to(TORCH[dtype])
    xr, normed = x.clone(), torch.empty_like(x)
    hm.residual_norm(xr, a, b, w, normed, 1e-5)
    want_x = oracle.to_bits((_f32(x) + _f32(a)) + _f32(b), dtype)
    ref_norm = torch.empty_like(x)
    hm.rmsnorm(ref_norm, xr, w, 1e-5)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(xr), want_x)
    assert torch.equal(normed, ref_norm)
    assert_close(oracle, host_f64(normed), oracle.rmsnorm(host_f64(xr), host_f64(w), 1e-5), dtype, "residual_norm")
    # one addend: the hm_residual_rmsnorm result; none: x untouched and the plain norm
    x1, n1, x2, n2 = x.clone(), torch.empty_like(x), x.clone(), torch.empty_like(x)
    hm.residual_norm(x1, a, None, w, n1, 1e-5)
    hm.residual_rmsnorm(x2, a, w, n2, 1e-5)
    x3, n3 = x.clone(), torch.empty_like(x)
    hm.residual_norm(x3, None, b, w, n3, 1e-5)
    n4 = torch.empty_like(x)
    hm.rmsnorm(n4, x, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(x1, x2) and torch.equal(n1, n2)
    assert torch.equal(x3, x) and torch.equal(n3, n4)


def _nonfinite_first(bits, dtype, sampled):
    # all exponent bits set, in the checked columns; the first in row-major order
    mask = 0x7C00 if dtype == "fp16" else 0x7F80
    hit = (bits & mask) == mask
    if sampled:
        hit[:, np.arange(bits.shape[1]) % 64 != 0] = False
    idx = np.flatnonzero(hit)
    return int(idx[0]) if idx.size else -1


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_find_nonfinite_device(oracle, hm, device, dtype):
    rng = np.random.default_rng(3)
    inf = 0x7C00 if dtype == "fp16" else 0x7F80
    nan = 0x7E00 if dtype == "fp16" else 0x7FC0
    for rows, cols in ((4, 256), (33, 4096), (2048, 4096)):
        base = oracle.to_bits(rng.standard_normal((rows, cols)).astype(np.float32), dtype)
        cases = [[]]
        for _ in range(3):
            cases.append([(int(rng.integers(rows)), int(rng.integers(cols)), int(rng.choice([inf, nan, 0x8000 | inf, 0xFFFF])))
                          for _ in range(int(rng.integers(1, 4)))])
        cases.append([(rows - 1, 64 * ((cols - 1) // 64), nan)])  # the last sampled column
        cases.append([(rows - 1, cols - 1, inf)])                 # the last element (unsampled)
        for plant in cases:
            bits = base.copy()
            for r, c, v in plant:
                bits[r, c] = v
            t = dev(bits.view(np.int16), device).view(TORCH[dtype])
            host = torch.from_numpy(bits.view(np.int16)).view(TORCH[dtype])
            for sampled in (False, True):
                want = _nonfinite_first(bits, dtype, sampled)
                assert hm.find_nonfinite(t, sampled) == want, (rows, cols, plant, sampled)
                assert hm.find_nonfinite(host, sampled) == want
    # a row view with a leading dimension larger than its width
    big = torch.zeros((8, 512), dtype=TORCH[dtype], device=device)
    big[5, 300] = float("nan")
    assert hm.find_nonfinite(big[:, :256]) == -1 and hm.find_nonfinite(big[:, 256:]) == 5 * 256 + 44
