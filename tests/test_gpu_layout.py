"""GPU: the one-time repack into the strip layout is bit-exact. Round trips through the C ABI, both input
routes (reference tiles, logical tensors) give the same bytes, and the device bytes decode with an
independent numpy reading of the layout."""

import numpy as np
import pytest
import torch

from gpu_util import copy_device_bytes, dev, dev_bits, host_bits, logical_to_device

pytestmark = pytest.mark.gpu


def decode_strips(quant, meta, k, n, group):
    """numpy reading of the strip layout: tile (s, t) at ((s * K/128 + t) * 64 + L) * 16, dword mu holds column
    16 s + (L & 15), K = 128 t + 32 mu + 8 (L >> 4) + e at nibble e/2 (even e) or 4 + e/2 (odd e); record
    ((s * K/128 + t) * 16 + col) * (128/g) + group in tile = scale | zero << 16."""
    words = quant.view(np.uint32).reshape(n // 16, k // 128, 64, 4)
    q = np.empty((k, n), np.uint8)
    nib = np.array([0, 4, 1, 5, 2, 6, 3, 7])
    for e in range(8):
        vals = (words >> (4 * nib[e])) & 0xF  # [s, t, L, mu]
        s_i, t_i, l_i, mu_i = np.indices(vals.shape)
        rows = 128 * t_i + 32 * mu_i + 8 * (l_i >> 4) + e
        cols = 16 * s_i + (l_i & 15)
        q[rows.ravel(), cols.ravel()] = vals.ravel()
    gpt = 128 // group
    rec = meta.view(np.uint32).reshape(n // 16, k // 128, 16, gpt)  # [strip][tile][column][group in tile]
    rec = rec.transpose(1, 3, 0, 2).reshape(k // group, n)
    scales = (rec & 0xFFFF).astype(np.uint16)
    zeros = (rec >> 16).astype(np.uint8)
    return q, scales, zeros


@pytest.mark.parametrize("k,n", [(128, 64), (384, 640), (256, 1152)])
def test_repack_from_tiles_round_trip(oracle, hm, device, k, n):
    rng = np.random.default_rng(k * 3 + n)
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.003, 0.25, 0, 16)
    tiles = dev(oracle.pack_tiles(q, s, z), device)
    w = hm.RepackedMatrix.from_tiles(tiles, k, n, dtype=torch.bfloat16)
    q2, s2, z2 = w.to_logical()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q2.cpu().numpy(), q)
    np.testing.assert_array_equal(host_bits(s2), s)
    np.testing.assert_array_equal(z2.cpu().numpy(), z)
    # the device bytes themselves, read by the layout's definition
    qp, qb, mp, mb = w.planes()
    dq, ds, dz = decode_strips(copy_device_bytes(qp, qb), copy_device_bytes(mp, mb), k, n, 128)
    np.testing.assert_array_equal(dq, q)
    np.testing.assert_array_equal(ds, s)
    np.testing.assert_array_equal(dz, z)


def test_repack_from_tiles_prefix_block(oracle, hm, device):
    # The leading [k, n] block of a larger packed matrix (hipkernels' packed_tiles_k / packed_tiles_n).
    rng = np.random.default_rng(21)
    K, N, k, n = 512, 1216, 256, 1152  # 19 tile columns in the full matrix
    q, s, z = oracle.random_weights(rng, K, N, 128, "bf16")
    w = hm.RepackedMatrix.from_tiles(dev(oracle.pack_tiles(q, s, z), device), K, N, k, n, dtype=torch.bfloat16)
    q2, s2, z2 = w.to_logical()
    np.testing.assert_array_equal(q2.cpu().numpy(), q[:k, :n])
    np.testing.assert_array_equal(host_bits(s2), s[: k // 128, :n])
    np.testing.assert_array_equal(z2.cpu().numpy(), z[: k // 128, :n])


def test_repack_from_tiles_to_fp16_scales(oracle, hm, device):
    # bf16 tile scales into an fp16 plane: round to nearest even (exact for normal-range scales).
    rng = np.random.default_rng(22)
    q, s, z = oracle.random_weights(rng, 256, 128, 128, "bf16", 1e-4, 0.5)
    w = hm.RepackedMatrix.from_tiles(dev(oracle.pack_tiles(q, s, z), device), 256, 128, dtype=torch.float16)
    _, s2, _ = w.to_logical()
    np.testing.assert_array_equal(host_bits(s2), oracle.f16_bits(oracle.bf16_bits_to_f32(s)))


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_repack_from_logical_round_trip(oracle, hm, device, group, dtype):
    rng = np.random.default_rng(group)
    k, n = 384, 272
    w_np = oracle.random_weights(rng, k, n, group, dtype)
    qd, sd, zd = logical_to_device(w_np, dtype, device)
    w = hm.RepackedMatrix.from_logical(qd, sd, zd, group, dtype=sd.dtype)
    q2, s2, z2 = w.to_logical()
    np.testing.assert_array_equal(q2.cpu().numpy(), w_np[0])
    np.testing.assert_array_equal(host_bits(s2), w_np[1])
    np.testing.assert_array_equal(z2.cpu().numpy(), w_np[2])
    qp, qb, mp, mb = w.planes()
    dq, ds, dz = decode_strips(copy_device_bytes(qp, qb), copy_device_bytes(mp, mb), k, n, group)
    np.testing.assert_array_equal(dq, w_np[0])
    np.testing.assert_array_equal(ds, w_np[1])
    np.testing.assert_array_equal(dz, w_np[2])


def test_tiles_and_logical_routes_give_identical_bytes(oracle, hm, device):
    rng = np.random.default_rng(23)
    k, n = 512, 640
    w_np = oracle.random_weights(rng, k, n, 128, "bf16")
    a = hm.RepackedMatrix.from_tiles(dev(oracle.pack_tiles(*w_np), device), k, n, dtype=torch.bfloat16)
    b = hm.RepackedMatrix.from_logical(*logical_to_device(w_np, "bf16", device), 128, dtype=torch.bfloat16)
    pa, pb = a.planes(), b.planes()
    assert pa[1] == pb[1] and pa[3] == pb[3]
    np.testing.assert_array_equal(copy_device_bytes(pa[0], pa[1]), copy_device_bytes(pb[0], pb[1]))
    np.testing.assert_array_equal(copy_device_bytes(pa[2], pa[3]), copy_device_bytes(pb[2], pb[3]))


def test_repack_rejects_bad_blocks(oracle, hm, device):
    tiles = torch.zeros(hm.packed_bytes(256, 128), dtype=torch.uint8, device=device)
    with pytest.raises(ValueError):
        hm.RepackedMatrix.from_tiles(tiles, 256, 128, 384, 128)
    with pytest.raises(ValueError):
        hm.RepackedMatrix.from_tiles(tiles, 256, 128, 256, 120)
    q = torch.zeros((256, 128), dtype=torch.uint8, device=device)
    s = torch.zeros((4, 128), dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        hm.RepackedMatrix.from_logical(q, s, q[:4], 48, dtype=torch.float16)
