"""GPU: the reference's fused-FFN inputs and its dequantize, through the C ABI.

- a gate_up tensor packed as one [H, 2 stored] matrix, interleaved per 64 channels or blocked (FfnSliceWeights.gate_up,
  kernels/gpu/include/heteromega/gpu_ffn.hpp:43-71; the FUSE_ACT GEMM's input, w4a16_gemm_packed.cu:549-578), built
  here with the reference's join (oracle.join_gate_up, pack_w4a16.cpp:80-88) and the reference packer: the layer
  from it gives the bits of the layer from separate gate and up matrices, and the SwiGLU projection on it the bits
  of hm_ffn_gate_up, both against the oracle too;
- hm_weights_dequantize, the counterpart of QuantizedLinearImpl::dequantize_packed (unified_llm_w4a16.cpp:710-790):
  bit for bit round((q - z) s);
- zero points outside 0..16 rejected at load."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, dev, dev_bits, host_bits, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu

HIDDEN, STORED = 1024, 2048


def _weights(oracle, dtype, seed, hidden=HIDDEN, inter=STORED):
    rng = np.random.default_rng(seed)
    return [oracle.random_weights(rng, hidden, inter, 128, dtype), oracle.random_weights(rng, hidden, inter, 128, dtype),
            oracle.random_weights(rng, inter, hidden, 128, dtype)]


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("layout", ["interleaved", "blocked"])
def test_ffn_from_gate_up_tiles_equals_two_matrix_route(oracle, hm, device, layout, dtype):
    gate, up, down = _weights(oracle, "bf16", 1)  # the 4352-byte tiles hold bf16 scales
    gu = dev(oracle.pack_tiles(*oracle.join_gate_up(gate, up, layout)), device)
    tiles = [dev(oracle.pack_tiles(*w), device) for w in (gate, up, down)]
    fused = hm.FfnLayer.from_gate_up_tiles(gu, tiles[2], HIDDEN, STORED, STORED, layout=layout, dtype=TORCH[dtype])
    separate = hm.FfnLayer.from_tiles(*tiles, HIDDEN, STORED, dtype=TORCH[dtype])
    # the prefix of the stored channels (FfnSliceWeights::prefix, gpu_ffn.hpp:66-70) against the same channels of the
    # full layer
    prefix = hm.FfnLayer.from_gate_up_tiles(gu, tiles[2], HIDDEN, 1536, STORED, layout=layout, dtype=TORCH[dtype])
    rng = np.random.default_rng(2)
    for m in (1, 5, 37, 256):
        x64, x = make_x(oracle, rng, m, HIDDEN, dtype, device)
        y_f = fused.forward(x)
        y_s = separate.forward(x)
        y_p = prefix.forward(x)
        y_s_part = separate.forward(x, channels=(0, 1536))
        torch.cuda.synchronize()
        assert torch.equal(y_f, y_s), (layout, dtype, m)
        assert torch.equal(y_p, y_s_part), (layout, dtype, m)
        # the tiles' bf16 scales become fp16 in an fp16 layer: the oracle takes the same rounded scales
        scaled = [(q, oracle.to_bits(oracle.bf16_bits_to_f32(s), dtype), z) for q, s, z in (gate, up, down)]
        ref, _ = oracle.ffn(x64, *scaled, 128, dtype)
        assert_close(oracle, host_f64(y_f), ref, dtype, f"gate_up tensor ({layout}) FFN M={m}")


@pytest.mark.parametrize("layout", ["interleaved", "blocked"])
def test_linear_swiglu_on_gate_up_tensor(oracle, hm, device, layout):
    gate, up, down = _weights(oracle, "bf16", 3)
    gu = dev(oracle.pack_tiles(*oracle.join_gate_up(gate, up, layout)), device)
    w = hm.RepackedMatrix.from_gate_up_tiles(gu, HIDDEN, STORED, layout=layout, dtype=torch.bfloat16)
    assert w.fused and w.n == 2 * STORED
    tiles = [dev(oracle.pack_tiles(*t), device) for t in (gate, up, down)]
    separate = hm.FfnLayer.from_tiles(*tiles, HIDDEN, STORED, dtype=torch.bfloat16)
    rng = np.random.default_rng(4)
    wg, wu = oracle.weights_f64(*gate, 128, "bf16"), oracle.weights_f64(*up, 128, "bf16")
    for m, ch in ((1, (0, STORED)), (16, (512, 1024)), (100, (0, STORED)), (300, (1024, 2048))):
        x64, x = make_x(oracle, rng, m, HIDDEN, "bf16", device)
        act = torch.empty((m, ch[1] - ch[0]), dtype=torch.bfloat16, device=device)
        hm.packed_linear_swiglu(act, x, w, channels=ch)
        act_ref = separate.gate_up(x, channels=ch)
        torch.cuda.synchronize()
        assert torch.equal(act, act_ref), (layout, m, ch)
        b, e = ch
        assert_close(oracle, host_f64(act), oracle.silu(x64 @ wg[:, b:e]) * (x64 @ wu[:, b:e]), "bf16", f"swiglu {layout} M={m}")
    # a fused matrix is not a plain projection
    with pytest.raises(ValueError):
        hm.packed_linear(torch.empty((1, 64), dtype=torch.bfloat16, device=device), x[:1], w, n=64)


@pytest.mark.parametrize("dtype,group", [("bf16", 128), ("fp16", 128), ("bf16", 64), ("fp16", 32)])
def test_dequantize_bit_exact(oracle, hm, device, dtype, group):
    rng = np.random.default_rng(5)
    k, n = 512, 384
    q, s, z = oracle.random_weights(rng, k, n, group, dtype)
    w = hm.RepackedMatrix.from_logical(*logical_to_device((q, s, z), dtype, device), group, dtype=TORCH[dtype])
    ref = oracle.to_bits(oracle.weights_f64(q, s, z, group, dtype).astype(np.float32), dtype)  # (q - z) s is exact in float32
    wt = w.dequantize(transposed=True)
    wn = w.dequantize(transposed=False)
    torch.cuda.synchronize()
    assert wt.shape == (n, k) and wn.shape == (k, n)
    np.testing.assert_array_equal(host_bits(wt), ref.T)
    np.testing.assert_array_equal(host_bits(wn), ref)


def test_dequantize_from_reference_tiles(oracle, hm, device):
    # dequantize_packed on the 4352-byte tiles: bf16 (w - z) * s, returned as [out, in]
    rng = np.random.default_rng(6)
    k, n = 384, 192
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16")
    w = hm.RepackedMatrix.from_tiles(dev(oracle.pack_tiles(q, s, z), device), k, n, dtype=torch.bfloat16)
    ref = oracle.bf16_bits((q.astype(np.float32) - np.repeat(z, 128, 0)) * np.repeat(oracle.bf16_bits_to_f32(s), 128, 0))
    np.testing.assert_array_equal(host_bits(w.dequantize()), ref.T)


def test_zero_points_outside_range_are_rejected(oracle, hm, device):
    rng = np.random.default_rng(7)
    k, n = 256, 128
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16")
    z16 = z.copy()
    z16[1, 5] = 16  # GPTQ's z after adding the one back: accepted
    hm.RepackedMatrix.from_logical(*logical_to_device((q, s, z16), "bf16", device), 128, dtype=torch.bfloat16)
    z17 = z.copy()
    z17[0, 3] = 17
    with pytest.raises(ValueError, match="zero points"):
        hm.RepackedMatrix.from_logical(*logical_to_device((q, s, z17), "bf16", device), 128, dtype=torch.bfloat16)
    tiles = oracle.pack_tiles(q, s, z)
    tiles[4224 + 3] = 200  # a zero byte the reference's GPU would read as -56
    with pytest.raises(ValueError, match="zero points"):
        hm.RepackedMatrix.from_tiles(dev(tiles, device), k, n, dtype=torch.bfloat16)
    down = oracle.random_weights(rng, n, k, 128, "bf16")  # [I, H] for the [H, I] = [k, n] gate and up
    with pytest.raises(ValueError, match="zero points"):
        hm.FfnLayer.from_logical(*[logical_to_device(w, "bf16", device) for w in ((q, s, z17), (q, s, z), down)], 128, dtype=torch.bfloat16)
