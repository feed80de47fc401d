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
        bufs = shim.gpu_ffn_slice_forward(gu, dt, 0, 1536, h, "interleaved", inter, x, y2, _stream())
        torch.cuda.synchronize()
        # GpuFfnBuffers::allocate's tensors as the reference sizes them (gpu_ffn.cpp:71-75); the engine's workspace
        # comes from gate_up's storage where that holds it (bufs[3] is the buffer grown otherwise)
        rows = -(-m // 128) * 128
        assert [tuple(b.shape) for b in bufs[:3]] == [(rows, 2 * 1536), (rows, 1536), (rows, h)]
        assert all(b.dtype == torch.bfloat16 for b in bufs[:3])
        del bufs
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


def _torch_logical(w, device=None):
    q, sb, z = w
    t = (torch.from_numpy(q.copy()), torch.from_numpy(sb.view(np.int16).copy()).view(torch.bfloat16), torch.from_numpy(z.astype(np.int8)))
    return tuple(x.to(device) for x in t) if device is not None else t


def test_packing_in_reference_form(oracle, hm, device, shim):
    # pack_w4a16 / pack_ffn_slice / slice_packed_ffn with the reference's torch signatures (gpu_ffn.hpp:27-98): the
    # packer gives the oracle's bytes; pack_ffn_slice packs the joined slices; slice_packed_ffn gathers whole tiles of
    # already packed matrices on the device and gives pack_ffn_slice's bytes (its contract, gpu_ffn.hpp:87-92).
    rng = np.random.default_rng(21)
    h, inter = 512, 1536
    gate, up = oracle.random_weights(rng, h, inter, 128, "bf16"), oracle.random_weights(rng, h, inter, 128, "bf16")
    down = oracle.random_weights(rng, inter, h, 128, "bf16")
    packed = shim.pack_w4a16(*_torch_logical(gate))
    assert packed.device.type == "cpu" and packed.dtype == torch.uint8
    assert np.array_equal(packed.numpy(), oracle.pack_tiles(*gate))
    assert np.array_equal(shim.pack_w4a16(*_torch_logical(gate, device)).numpy(), oracle.pack_tiles(*gate))  # device inputs too
    quant = [*_torch_logical(gate), *_torch_logical(up), *_torch_logical(down)]
    gt, ut, dt = (dev(oracle.pack_tiles(*w), device) for w in (gate, up, down))
    for layout in ("blocked", "interleaved"):
        for begin, end in ((0, inter), (512, 1536), (0, 640), (1024, 1152)):
            gu, dn, b, e, hid = shim.pack_ffn_slice(quant, begin, end, layout)
            assert (b, e, hid) == (begin, end, h)
            sl = lambda w: tuple(a[:, begin:end] for a in w)
            want_gu = oracle.pack_tiles(*oracle.join_gate_up(sl(gate), sl(up), layout))
            want_dn = oracle.pack_tiles(down[0][begin:end], down[1][begin // 128:end // 128], down[2][begin // 128:end // 128])
            assert np.array_equal(gu.numpy(), want_gu) and np.array_equal(dn.numpy(), want_dn), (layout, begin, end)
            sgu, sdn, _, _, _ = shim.slice_packed_ffn(gt, ut, dt, h, inter, begin, end, layout, "")
            assert sgu.is_cuda and np.array_equal(sgu.cpu().numpy(), want_gu) and np.array_equal(sdn.cpu().numpy(), want_dn)
            if (begin, end) == (0, inter):
                assert sdn.data_ptr() == dt.data_ptr()  # the whole range keeps down itself
    # FfnSliceWeights::to: CPU packed matrices sliced, then moved
    cgu, cdn, _, _, _ = shim.slice_packed_ffn(gt.cpu(), ut.cpu(), dt.cpu(), h, inter, 512, 1024, "interleaved", str(device))
    assert cgu.is_cuda and cdn.is_cuda
    with pytest.raises(RuntimeError):
        shim.slice_packed_ffn(gt, ut, dt, h, inter, 100, 1024, "blocked", "")
    with pytest.raises(RuntimeError):
        shim.pack_w4a16(*_torch_logical(oracle.random_weights(rng, 128, 96, 128, "bf16")))


def test_layer_boundary_in_reference_form(oracle, hm, device, shim):
    # residual_add2 (bf16 and fp32 partials) and residual_norm_bf16 with the reference's argument order
    # (gpu_ffn.hpp:132-163), bit for bit against the engine's own entry points; the GEMMs after the boundary read
    # the normalized rows and count as GemmInputReuse hits, as the reference's Q/K/V do (unified_llm_w4a16.cpp:2529-2566).
    rng = np.random.default_rng(22)
    m, h = 32, 1024
    _, x = make_x(oracle, rng, m, h, "bf16", device)
    _, g = make_x(oracle, rng, m, h, "bf16", device, 0.4)
    n32 = torch.from_numpy((rng.standard_normal((m, h)) * 0.4).astype(np.float32)).to(device)
    for yn in (g.clone().flip(0), n32):
        a, b = x.clone(), x.clone()
        shim.residual_add2(a, g, yn, _stream())
        hm.residual_add2(b, g, yn)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    assert shim.residual_norm_supports(m, h) and not shim.residual_norm_supports(0, h) and not shim.residual_norm_supports(m, 1001)
    w = (torch.rand((h,), device=device) + 0.5).to(torch.bfloat16)
    mats = [_tiles(oracle, rng, h, 512, device)[1] for _ in range(3)]
    xa, gemm_x, normed = x.clone(), torch.empty_like(x), torch.empty_like(x)
    hits, outs = shim.residual_norm_bf16(xa, g, g.flip(0).contiguous(), w, normed, gemm_x, 1e-5, _stream(), mats, 512)
    xb, nb = x.clone(), torch.empty_like(x)
    hm.residual_norm(xb, g, g.flip(0).contiguous(), w, nb, 1e-5)
    torch.cuda.synchronize()
    assert hits == 3
    assert torch.equal(xa, xb) and torch.equal(gemm_x, nb) and torch.equal(normed, nb)
    for wt, out in zip(mats, outs):
        ref = torch.empty_like(out)
        shim.gemm_w4a16(ref, nb, wt, h, 512, h, 512, _stream())
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    # without normed (the reference's row-order buffer) only gemm_x is written; no GEMM, no hits
    xc, gx = x.clone(), torch.empty_like(x)
    hits, _ = shim.residual_norm_bf16(xc, g, None, w, None, gx, 1e-5, _stream(), [], 512)
    xd, nd = x.clone(), torch.empty_like(x)
    hm.residual_norm(xd, g, None, w, nd, 1e-5)
    torch.cuda.synchronize()
    assert hits == 0 and torch.equal(xc, xd) and torch.equal(gx, nd)
    with pytest.raises(RuntimeError):
        shim.gemm_input_buffers(m, h, _stream())
    assert shim.configured_gemm_kernel() in ("fast", "mosaic")
    t = torch.zeros(8, dtype=torch.uint8, device=device)
    assert shim.gemm_uncached_weights(t).data_ptr() == t.data_ptr()


def test_finite_check_in_reference_form(device, shim):
    # parse_finite_check / find_nonfinite_bf16 on the reference's own cases (tests/ffn_deploy/contract_test.cpp:100-124),
    # and the device scan of the same data.
    assert shim.parse_finite_check("", True) == "full" and shim.parse_finite_check("", False) == "full"
    assert shim.parse_finite_check("full", False) == "full" and shim.parse_finite_check("sampled", False) == "sampled"
    with pytest.raises(ValueError):
        shim.parse_finite_check("off", False)
    rows, cols = 4, 256
    bits = np.full((rows, cols), 0x3F80, np.uint16)
    first = torch.empty((1,), dtype=torch.int64, device=device)

    def both(sampled):
        host = torch.from_numpy(bits.view(np.int16).copy())
        shim.find_nonfinite_device(host.view(torch.bfloat16).to(device), sampled, first, _stream())
        torch.cuda.synchronize()
        got = shim.find_nonfinite_bf16(host, sampled)
        assert int(first.item()) == got
        return got

    assert both(False) == -1 and both(True) == -1
    for v in (0x7F80, 0xFF80, 0x7FC0, 0xFFFF):
        bits[2, 3] = v
        assert both(False) == 2 * cols + 3 and both(True) == -1
        bits[2, 3] = 0x3F80
        bits[3, 64] = v
        assert both(True) == 3 * cols + 64
        bits[3, 64] = 0x3F80
    bits[1, :] = 0x7FC0
    assert both(False) == cols and both(True) == cols


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused first call leaves its capture empty
def test_repacked_copy_follows_the_tensor(oracle, hm, device, shim):
    # A repacked copy is used only while its packed tensor's storage lives unchanged: weights freed and replaced by
    # others at the same address, or rewritten in place, are repacked on the next call (not served from the old copy).
    rng = np.random.default_rng(23)
    k, n = 1024, 512
    wa, wb = oracle.random_weights(rng, k, n, 128, "bf16"), oracle.random_weights(rng, k, n, 128, "bf16")
    _, x = make_x(oracle, rng, 1, k, "bf16", device)
    ref_b = torch.empty((1, n), dtype=torch.bfloat16, device=device)
    hm.packed_linear(ref_b, x, hm.RepackedMatrix.from_tiles(dev(oracle.pack_tiles(*wb), device), k, n))
    out = torch.empty((1, n), dtype=torch.bfloat16, device=device)
    a = dev(oracle.pack_tiles(*wa), device)
    shim.w4a16_gemv_fused_packed(out, x, a, k, n, -1, 0, _stream())
    torch.cuda.synchronize()
    ref_a = out.clone()
    assert not torch.equal(ref_a, ref_b)
    addr = a.data_ptr()
    del a
    b = dev(oracle.pack_tiles(*wb), device)  # the caching allocator hands out the freed block again
    shim.w4a16_gemv_fused_packed(out, x, b, k, n, -1, 0, _stream())
    torch.cuda.synchronize()
    print("same address reused:", b.data_ptr() == addr)
    assert torch.equal(out, ref_b)
    # rewritten in place: the version counter moves, the next call repacks
    b.copy_(dev(oracle.pack_tiles(*wa), device))
    shim.w4a16_gemv_fused_packed(out, x, b, k, n, -1, 0, _stream())
    torch.cuda.synchronize()
    assert torch.equal(out, ref_a)
    # unchanged: the copy is reused, also under graph capture; a first call under capture is refused
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    out2 = torch.empty_like(out)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            shim.w4a16_gemv_fused_packed(out2, x, b, k, n, -1, 0, s.cuda_stream)
    for _ in range(3):
        out2.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, ref_a)
    fresh = dev(oracle.pack_tiles(*wb), device)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="capture"):
        with torch.cuda.stream(s):
            with torch.cuda.graph(g2, stream=s):
                shim.w4a16_gemv_fused_packed(out2, x, fresh, k, n, -1, 0, s.cuda_stream)
    torch.cuda.synchronize()
