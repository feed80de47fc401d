"""GPU: the reference's C++ operator signatures (heteromega_amd/shim/hm_reference_api.hpp, compiled against torch's
C++ headers) called with torch tensors, as a C++ caller of the reference would call them. Each gives the bits of the
engine's own entry point for the same work, and the oracle's values within tolerance."""

import numpy as np
import pytest
import torch

from gpu_util import assert_close, dev, host_f64, make_x

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def shim(hm):
    from heteromega_amd import _reference_shim

    return _reference_shim


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _tiles(oracle, rng, k, n, device, dtype="bf16"):
    w = oracle.random_weights(rng, k, n, 128, dtype)
    return w, dev(oracle.pack_tiles(*w), device)


def test_hipkernels_gemv_and_gemm(oracle, hm, device, shim):
    rng = np.random.default_rng(1)
    k, total_n = 2048, 3072
    w, tiles = _tiles(oracle, rng, k, total_n, device)
    rw = hm.RepackedMatrix.from_tiles(tiles, k, total_n)
    wf = oracle.weights_f64(*w, 128, "bf16")
    # GEMV over columns [start_col, start_col + n) of the whole matrix (w4a16_gemv_packed.cu:178-194)
    x64, x = make_x(oracle, rng, 1, k, "bf16", device)
    for n, start in ((1024, 0), (512, 1536), (3072, 0)):
        out = torch.empty((1, n), dtype=torch.bfloat16, device=device)
        shim.w4a16_gemv_fused_packed(out, x, tiles, k, n, total_n, start, _stream())
        ref = torch.empty_like(out)
        hm.packed_linear(ref, x, rw, n=n, col_begin=start)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert_close(oracle, host_f64(out), x64 @ wf[:, start:start + n], "bf16", f"shim gemv n={n} start={start}")
    # GEMM on the whole matrix and on a leading block of it (w4a16_gemm_fused_packed[_tiles])
    x64, x = make_x(oracle, rng, 64, k, "bf16", device)
    out = torch.empty((64, total_n), dtype=torch.bfloat16, device=device)
    shim.w4a16_gemm_fused_packed(out, x, tiles, k, total_n, _stream())
    ref = torch.empty_like(out)
    hm.packed_linear(ref, x, rw)
    blk = torch.empty((64, 1024), dtype=torch.bfloat16, device=device)
    shim.w4a16_gemm_fused_packed_tiles(blk, x[:, :1024].contiguous(), tiles, 1024, 1024, k // 128, total_n // 64, _stream(), False)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert_close(oracle, host_f64(blk), x64[:, :1024] @ wf[:1024, :1024], "bf16", "shim gemm leading block")
    # heteromega::gemv_w4a16 / gemm_w4a16 / packed_linear on the same matrix
    for m in (1, 40):
        x64, x = make_x(oracle, rng, m, k, "bf16", device)
        a = torch.empty((m, 2048), dtype=torch.bfloat16, device=device)
        (shim.gemv_w4a16(a, x, tiles, k, 2048, k, total_n, 0, _stream()) if m == 1 else
         shim.gemm_w4a16(a, x, tiles, k, 2048, k, total_n, _stream()))
        b = torch.empty_like(a)
        shim.packed_linear(b, x, tiles, k, 2048, _stream(), k, total_n, False)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        assert_close(oracle, host_f64(a), x64 @ wf[:, :2048], "bf16", f"shim heteromega linear M={m}")
    assert shim.gemm_w4a16_supports(40, 2048, 2048) and not shim.gemm_w4a16_supports(40, 2000, 2048)


def test_fused_gate_up_paths(oracle, hm, device, shim):
    # fuse_activation = true on the reference's interleaved gate_up (w4a16_gemm_packed.cu:549-578), gemm_w4a16_ffn,
    # gpu_ffn_slice_forward with a prefix, silu_mul and GpuFfnModel, each against the engine's own route.
    rng = np.random.default_rng(2)
    h, inter = 1024, 2048
    gate, gt = _tiles(oracle, rng, h, inter, device)
    up, ut = _tiles(oracle, rng, h, inter, device)
    down, dt = _tiles(oracle, rng, inter, h, device)
    gu = dev(oracle.pack_tiles(*oracle.join_gate_up(gate, up, "interleaved")), device)
    layer = hm.FfnLayer.from_tiles(gt, ut, dt, h, inter)
    for m in (1, 16, 96):
        x64, x = make_x(oracle, rng, m, h, "bf16", device)
        act = torch.empty((m, inter), dtype=torch.bfloat16, device=device)
        shim.w4a16_gemm_fused_packed_tiles(act, x, gu, h, 2 * inter, h // 128, 2 * inter // 64, _stream(), True)
        act2 = torch.empty_like(act)
        shim.packed_linear(act2, x, gu, h, 2 * inter, _stream(), 0, 0, True)
        y = torch.empty((m, h), dtype=torch.bfloat16, device=device)
        shim.gemm_w4a16_ffn(y, x, gu, dt, h, 1536, inter, _stream())
        y2 = torch.empty_like(y)
        ws = shim.gpu_ffn_slice_forward(gu, dt, 0, 1536, h, "interleaved", inter, x, y2, _stream())
        torch.cuda.synchronize()
        del ws
        assert torch.equal(act, layer.gate_up(x))
        assert torch.equal(act2, act)
        y_ref = layer.forward(x, channels=(0, 1536))
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref) and torch.equal(y2, y_ref)
        ref, _ = oracle.ffn(x64, gate, up, down, 128, "bf16", channels=(0, 1536))
        assert_close(oracle, host_f64(y), ref, "bf16", f"shim gemm_w4a16_ffn M={m}")
    # silu_mul on an interleaved gate_up activation
    gu_act = torch.randn((8, 2 * 256), device=device).to(torch.bfloat16)
    a1 = torch.empty((8, 256), dtype=torch.bfloat16, device=device)
    a2 = torch.empty_like(a1)
    shim.silu_mul(gu_act, a1, _stream(), "interleaved")
    hm.silu_mul(gu_act, a2, layout="interleaved")
    # GpuFfnModel with the reference's add_layer signature (gpu_ffn.hpp:223)
    model = shim.GpuFfnModel()
    model.add_layer(gt, ut, dt, h, inter)
    model.set_split(inter, 1024)
    assert model.layers() == 1 and model.channels(1) == 1024 and model.channels(8) == inter
    x64, x = make_x(oracle, rng, 1, h, "bf16", device)
    y = torch.empty((1, h), dtype=torch.bfloat16, device=device)
    model.forward(0, x, y, _stream())
    torch.cuda.synchronize()
    assert torch.equal(a1, a2)
    assert torch.equal(y, layer.forward(x, channels=(0, 1024)))
    # argument errors surface as torch errors (TORCH_CHECK), as in the reference
    with pytest.raises(RuntimeError):
        model.set_split(100, 1024)
