"""CPU checks of the C ABI: the library loads, exports every symbol of include/hm_w4a16.h, and its host-only
entry points (tile packer, tile index, AWQ unpack, partition descriptor, argument validation) agree with the
oracle. No GPU compute is called here."""

import ctypes
import json
import os
import re

import numpy as np
import torch
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "known_answers.json")))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "hm_w4a16.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = _declared_symbols()
    for must in ("hm_ffn_forward", "hm_linear", "hm_weights_from_tiles", "hm_pack_w4a16", "hm_last_error"):
        assert must in syms


def test_library_exports_every_declared_symbol(hm):
    from heteromega_amd import _lib

    L = _lib.load()
    missing = [s for s in _declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    assert L.hm_abi_version() == 1


def test_python_binding_covers_every_symbol():
    from heteromega_amd import _lib

    assert set(_declared_symbols()) == set(_lib._SIGNATURES)


def test_pack_w4a16_matches_oracle(hm, oracle):
    rng = np.random.default_rng(0)
    for k, n in [(128, 64), (384, 640), (256, 1152)]:
        q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.002, 0.02, 6, 10)
        np.testing.assert_array_equal(hm.pack_w4a16(q, s, z.astype(np.int8)), oracle.pack_tiles(q, s, z))


def test_pack_w4a16_rejects_bad_shapes(hm):
    with pytest.raises(ValueError):
        hm.pack_w4a16(np.zeros((128, 96), np.uint8), np.zeros((1, 96), np.uint16), np.zeros((1, 96), np.int8))
    with pytest.raises(ValueError):
        hm.pack_w4a16(np.zeros((100, 64), np.uint8), np.zeros((1, 64), np.uint16), np.zeros((1, 64), np.int8))


def test_packed_bytes_contract(hm):
    ka = GOLDEN["contract_sizes"]
    assert hm.packed_bytes(ka["hidden"], ka["intermediate"]) == ka["weight_bytes"]
    assert hm.packed_bytes(100, 64) == -1


def test_tile_index_matches_oracle(hm, oracle):
    for tk, tn in [(3, 10), (32, 224), (2, 19)]:
        for c in range(tn):
            for r in range(tk):
                assert hm.packed_tile_index(c, r, tk, tn) == oracle.tile_index(c, r, tk, tn)
    with pytest.raises(ValueError):
        hm.packed_tile_index(10, 0, 3, 10)


def test_awq_unpack_matches_oracle(hm, oracle):
    rng = np.random.default_rng(1)
    packed = rng.integers(-2 ** 31, 2 ** 31, (8, 32), dtype=np.int64).astype(np.int32)
    np.testing.assert_array_equal(hm.awq_unpack_qweight(packed), oracle.awq_unpack(packed))


def test_partition_known_answers(hm):
    ka = GOLDEN["partition_from_ratio"]
    for inter, ratio, align, exp in ka["cases"]:
        assert hm.FFNPartition.from_ratio(inter, ratio, align).npu_channels == exp
    for r in ka["rejected_ratios"]:
        with pytest.raises(ValueError):
            hm.FFNPartition.from_ratio(32, float(r), 4)
    for args in GOLDEN["partition_rejects"]["cases"]:
        with pytest.raises(ValueError):
            hm.FFNPartition(*args)
    with pytest.raises(ValueError):
        hm.FFNPartition(32, 4.0, 4)
    p = hm.FFNPartition(14336, 4352)
    assert p.slices == {"npu": (0, 4352), "gpu": (4352, 14336)}
    assert hm.FFNPartition(14336, 0).slices["gpu"] == (0, 14336)


def test_invalid_arguments_are_reported_not_fatal(hm):
    from heteromega_amd import _lib

    L = _lib.load()
    out = ctypes.c_void_p()
    # null source, bad shapes, bad dtype: status + message, no crash, no device work
    assert L.hm_weights_from_tiles(None, 4096, 14336, 4096, 14336, 0, None, ctypes.byref(out)) == _lib.HM_INVALID_ARGUMENT
    assert "null" in _lib.last_error()
    fake = ctypes.c_void_p(0x1000)
    assert L.hm_weights_from_tiles(fake, 4000, 14336, 4000, 14336, 0, None, ctypes.byref(out)) == _lib.HM_INVALID_ARGUMENT
    assert L.hm_weights_from_tiles(fake, 4096, 14336, 4096, 14336, 7, None, ctypes.byref(out)) == _lib.HM_INVALID_ARGUMENT
    assert L.hm_weights_from_logical(fake, fake, fake, 4096, 4096, 48, 1, None, ctypes.byref(out)) == _lib.HM_INVALID_ARGUMENT
    assert "group" in _lib.last_error()
    assert L.hm_ffn_forward(None, fake, 4096, fake, 4096, 1, 0, 128, None, 0, None) == _lib.HM_INVALID_ARGUMENT
    assert L.hm_linear(None, fake, 16, fake, 16, 1, 128, 16, 0, None, 0, None) == _lib.HM_INVALID_ARGUMENT
    assert L.hm_silu_mul(fake, 16, fake, 8, 1, 8, 5, 0, None) == _lib.HM_INVALID_ARGUMENT
    assert L.hm_weights_destroy(None) == _lib.HM_OK
    assert L.hm_ffn_destroy(None) == _lib.HM_OK


def test_product_does_not_import_oracle():
    # The product package must not route through the CPU oracle.
    for dirpath, _, files in os.walk(os.path.join(ROOT, "heteromega_amd")):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("oracle/_ref", ""), f


def test_pack_w4a16_rejects_zero_points_outside_range(hm):
    import ctypes

    import numpy as np

    lib = hm._lib.load()
    k, n = 128, 64
    q = np.zeros((k, n), np.uint8)
    s = np.full((1, n), 0x3C00, np.uint16)
    out = np.empty(hm.packed_bytes(k, n), np.uint8)
    for zv, ok in ((16, True), (17, False), (-1, False), (0, True)):
        z = np.zeros((1, n), np.int8)
        z[0, 7] = zv
        st = lib.hm_pack_w4a16(q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p), z.ctypes.data_as(ctypes.c_void_p), k, n,
                               out.ctypes.data_as(ctypes.c_void_p))
        assert (st == hm._lib.HM_OK) == ok, (zv, st)
        if not ok:
            assert "zero point" in hm._lib.last_error()


def test_reference_shim_loads_and_checks_arguments(hm):
    # The reference-signature C++ operators compile against torch's headers and load; argument errors are torch
    # errors before anything touches a GPU.
    import torch

    from heteromega_amd import _reference_shim as shim

    for name in ("w4a16_gemm_fused_packed", "w4a16_gemm_fused_packed_tiles", "w4a16_gemv_fused_packed", "gemv_w4a16", "gemm_w4a16",
                 "gemm_w4a16_ffn", "silu_mul", "packed_linear", "gpu_ffn_slice_forward", "GpuFfnModel"):
        assert hasattr(shim, name), name
    assert shim.gemm_w4a16_supports(17, 4096, 14336) and not shim.gemm_w4a16_supports(17, 4096, 100)
    assert shim.gemm_w4a16_ffn_supports(1, 4096, 14336) and not shim.gemm_w4a16_ffn_supports(1, 4000, 14336)
    x = torch.zeros((1, 128), dtype=torch.bfloat16)
    out = torch.zeros((1, 64), dtype=torch.bfloat16)
    packed = torch.zeros(4352, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="device uint8"):
        shim.w4a16_gemv_fused_packed(out, x, packed, 128, 64, -1, 0, 0)


def test_find_nonfinite_host_known_answers(hm):
    # The reference's own cases for find_nonfinite_bf16 (tests/ffn_deploy/contract_test.cpp:107-124): bf16 1.0 everywhere,
    # one nonfinite value at an unsampled and at a sampled column, then a whole nonfinite row. Host scan, no GPU.
    rows, cols = 4, 256
    bits = np.full((rows, cols), 0x3F80, np.uint16)
    t = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    assert hm.find_nonfinite(t(bits)) == -1 and hm.find_nonfinite(t(bits), sampled=True) == -1
    for nonfinite in (0x7F80, 0xFF80, 0x7FC0, 0xFFFF):
        bits[2, 3] = nonfinite
        assert hm.find_nonfinite(t(bits)) == 2 * cols + 3
        assert hm.find_nonfinite(t(bits), sampled=True) == -1
        bits[2, 3] = 0x3F80
        bits[3, 64] = nonfinite
        assert hm.find_nonfinite(t(bits), sampled=True) == 3 * cols + 64
        bits[3, 64] = 0x3F80
    bits[1, :] = 0x7FC0
    assert hm.find_nonfinite(t(bits)) == cols and hm.find_nonfinite(t(bits), sampled=True) == cols
    # fp16: the exponent field is bits 10..14; the largest finite value and a subnormal are finite
    h = np.full((2, 8), 0x3C00, np.uint16)
    h[0, 1], h[0, 2] = 0x7BFF, 0x0001
    f16 = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.float16)
    assert hm.find_nonfinite(f16(h)) == -1
    h[1, 5] = 0xFC00
    assert hm.find_nonfinite(f16(h)) == 8 + 5
    assert hm.kFiniteSampleStride == 64
