"""CPU: the reference's own packing code (kernels/gpu/src/pack_w4a16.cpp, built from its sources into oracle/_ref by
oracle/build_ref.py) against the oracle's restatement, the engine's host packer (hm_pack_w4a16) and the shim's torch-form
pack_ffn_slice / slice_packed_ffn: byte for byte. Skipped where the reference's build is absent."""

import ctypes
import os

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "libref_pack.so")

pytestmark = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref/libref_pack.so not built (oracle/build_ref.py)")


@pytest.fixture(scope="module")
def ref():
    lib = ctypes.CDLL(REF)
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    lib.ref_pack_w4a16.argtypes = [P, P, P, I64, I64, P]
    lib.ref_packed_tile_index.argtypes = [I64, I64, I64, I64]
    lib.ref_packed_tile_index.restype = I64
    lib.ref_pack_ffn_slice.argtypes = [P] * 9 + [I64, I64, I64, I64, ctypes.c_int, P, P]
    lib.ref_slice_packed_ffn.argtypes = [P, P, P, I64, I64, I64, I64, ctypes.c_int, P, P]
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _ref_pack(ref, q, s, z):
    k, n = q.shape
    out = np.empty((k // 128) * (n // 64) * 4352, np.uint8)
    assert ref.ref_pack_w4a16(_p(q), _p(s), _p(z.astype(np.int8)), k, n, _p(out)) == 0
    return out


def test_reference_packer_pins_oracle_and_engine(ref, oracle, hm):
    rng = np.random.default_rng(31)
    for k, n, zlo, zhi in [(128, 64, 0, 16), (384, 640, 0, 16), (256, 1152, 6, 10), (1024, 512, 15, 16), (512, 64, 0, 1)]:
        q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.001, 0.02, zlo, zhi)
        want = _ref_pack(ref, q, s, z)
        assert np.array_equal(oracle.pack_tiles(q, s, z), want), (k, n)
        assert np.array_equal(oracle.pack_tiles_literal(q, s, z), want), (k, n)
        assert np.array_equal(hm.pack_w4a16(q, s, z.astype(np.int8)), want), (k, n)
    # scales of every bf16 bit pattern class (signs, subnormals, inf) pass through the tiles unchanged
    q = rng.integers(0, 16, (128, 64), dtype=np.uint8)
    s = rng.integers(0, 1 << 16, (1, 64), dtype=np.uint16)
    z = rng.integers(0, 16, (1, 64), dtype=np.uint8)
    assert np.array_equal(hm.pack_w4a16(q, s, z.astype(np.int8)), _ref_pack(ref, q, s, z))


def test_reference_tile_index(ref, oracle, hm):
    for tk, tn in [(1, 1), (3, 10), (32, 224), (2, 19), (112, 64)]:
        for c in range(tn):
            for r in range(tk):
                want = ref.ref_packed_tile_index(c, r, tk, tn)
                assert oracle.tile_index(c, r, tk, tn) == want and hm.packed_tile_index(c, r, tk, tn) == want


def test_reference_slicers_pin_the_shim(ref, oracle, hm):
    from heteromega_amd import _reference_shim as shim

    rng = np.random.default_rng(32)
    h, inter = 256, 1024
    gate, up = oracle.random_weights(rng, h, inter, 128, "bf16"), oracle.random_weights(rng, h, inter, 128, "bf16")
    down = oracle.random_weights(rng, inter, h, 128, "bf16")
    quant = []
    for q, s, z in (gate, up, down):
        quant += [torch.from_numpy(q.copy()), torch.from_numpy(s.view(np.int16).copy()).view(torch.bfloat16), torch.from_numpy(z.astype(np.int8))]
    gt, ut, dt = (oracle.pack_tiles(*w) for w in (gate, up, down))
    args9 = [gate[0], gate[1], gate[2].astype(np.int8), up[0], up[1], up[2].astype(np.int8), down[0], down[1], down[2].astype(np.int8)]
    for layout in ("blocked", "interleaved"):
        for begin, end in ((0, inter), (256, 768), (512, 640)):
            n = end - begin
            gu = np.empty((h // 128) * (2 * n // 64) * 4352, np.uint8)
            dn = np.empty((n // 128) * (h // 64) * 4352, np.uint8)
            assert ref.ref_pack_ffn_slice(*[_p(a) for a in args9], h, inter, begin, end, int(layout == "interleaved"), _p(gu), _p(dn)) == 0
            sgu, sdn, _, _, _ = shim.pack_ffn_slice(quant, begin, end, layout)
            assert np.array_equal(sgu.numpy(), gu) and np.array_equal(sdn.numpy(), dn), (layout, begin, end)
            gu2, dn2 = np.empty_like(gu), np.empty_like(dn)
            assert ref.ref_slice_packed_ffn(_p(gt), _p(ut), _p(dt), h, inter, begin, end, int(layout == "interleaved"), _p(gu2), _p(dn2)) == 0
            assert np.array_equal(gu2, gu) and np.array_equal(dn2, dn)  # the reference's own equality (gpu_ffn.hpp:87-92)
            cgu, cdn, _, _, _ = shim.slice_packed_ffn(*(torch.from_numpy(a) for a in (gt, ut, dt)), h, inter, begin, end, layout, "")
            assert np.array_equal(cgu.numpy(), gu) and np.array_equal(cdn.numpy(), dn), (layout, begin, end)
