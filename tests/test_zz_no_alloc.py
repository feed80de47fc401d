"""GPU: hm_ffn_forward_static (the FFN forward on the library's static device scratch, no workspace argument)
gives the bits of hm_ffn_forward with a caller workspace, call after call with shrinking inputs (at the benchmark
shapes and at seeded random ones), and rejects requests larger than its scratch before launching anything."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import TORCH, logical_to_device, make_x

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20  # HM_STATIC_SCRATCH_BYTES in include/hm_w4a16.h


def _layer(oracle, hm, device, hidden, inter, group, dtype, seed):
    rng = np.random.default_rng(seed)
    ws = [oracle.random_weights(rng, hidden, inter, group, dtype), oracle.random_weights(rng, hidden, inter, group, dtype),
          oracle.random_weights(rng, inter, hidden, group, dtype)]
    return hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in ws), group, dtype=TORCH[dtype])


def _static(hm, layer, y, x, m, ch):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return hm._lib.load().hm_ffn_forward_static(layer._h, ctypes.c_void_p(y.data_ptr()), y.stride(0), ctypes.c_void_p(x.data_ptr()),
                                                x.stride(0), m, ch[0], ch[1], stream)


@pytest.mark.parametrize("shape", [(4096, 14336, 128, "fp16"), (5120, 13824, 64, "bf16")])
def test_static_scratch_forward_equals_workspace_forward(oracle, hm, device, shape):
    hidden, inter, group, dtype = shape
    layer = _layer(oracle, hm, device, hidden, inter, group, dtype, 3)
    lib = hm._lib.load()
    need16 = lib.hm_ffn_workspace_bytes(layer._h, 16)
    print(f"{hidden}x{inter} g={group}: workspace for 16 rows = {need16} bytes", flush=True)
    assert need16 <= SCRATCH_BYTES
    rng = np.random.default_rng(5)
    ch_half = (inter // 256) * 128
    # Two calls in a row with shrinking inputs (the second reuses the scratch the first left behind), then a
    # channel range and one row.
    for m, ch in ((16, (0, inter)), (4, (0, inter)), (16, (ch_half, inter)), (1, (0, inter)), (1, (0, ch_half))):
        _, x = make_x(oracle, rng, m, hidden, dtype, device)
        y_static = torch.full((m, hidden), float("nan"), dtype=TORCH[dtype], device=device)
        print(f"static forward m={m} channels={ch}", flush=True)
        hm._lib.check(_static(hm, layer, y_static, x, m, ch))
        y_ws = layer.forward(x, channels=ch)
        torch.cuda.synchronize()
        assert torch.equal(y_static, y_ws), (m, ch)


def test_static_scratch_rejects_large_requests(oracle, hm, device):
    layer = _layer(oracle, hm, device, 1024, 2048, 128, "fp16", 4)
    lib = hm._lib.load()
    m = 64  # prefill rows reserve the GEMM's split partials (32 MiB): more than the static scratch
    assert lib.hm_ffn_workspace_bytes(layer._h, m) > SCRATCH_BYTES
    x = torch.zeros((m, 1024), dtype=torch.float16, device=device)
    y = torch.zeros((m, 1024), dtype=torch.float16, device=device)
    assert _static(hm, layer, y, x, m, (0, 2048)) == hm._lib.HM_WORKSPACE_TOO_SMALL
    assert "static" in hm._lib.last_error()
    assert _static(hm, layer, y, x, 0, (0, 2048)) == hm._lib.HM_INVALID_ARGUMENT


def test_static_scratch_random_shapes(oracle, hm, device):
    # Seeded random layers and calls (1..16 rows, channel ranges, groups 32 / 64 / 128, both dtypes), one after
    # another on the shared scratch: each call's bits equal hm_ffn_forward's with a caller workspace, and a call
    # whose workspace would exceed the scratch is refused with HM_WORKSPACE_TOO_SMALL.
    rng = np.random.default_rng(20261206)
    lib = hm._lib.load()
    for case in range(12):
        group = int(rng.choice([32, 64, 128]))
        dtype = str(rng.choice(["fp16", "bf16"]))
        hidden = 128 * int(rng.integers(1, 26))
        inter = 128 * int(rng.integers(1, min(49, (6 << 20) // (hidden * 128)) + 1))
        layer = _layer(oracle, hm, device, hidden, inter, group, dtype, 100 + case)
        for m in sorted((int(v) for v in rng.integers(1, 17, 2)), reverse=True):
            b = 128 * int(rng.integers(0, inter // 128)) if rng.random() < 0.4 else 0
            e = b + 128 * int(rng.integers(1, (inter - b) // 128 + 1)) if rng.random() < 0.5 else inter
            _, x = make_x(oracle, rng, m, hidden, dtype, device)
            y_static = torch.full((m, hidden), float("nan"), dtype=TORCH[dtype], device=device)
            print(f"static forward case {case}: {hidden}x{inter} g={group} {dtype} m={m} channels=({b}, {e})", flush=True)
            rc = _static(hm, layer, y_static, x, m, (b, e))
            if lib.hm_ffn_workspace_bytes(layer._h, m) > SCRATCH_BYTES:
                assert rc == hm._lib.HM_WORKSPACE_TOO_SMALL
                continue
            hm._lib.check(rc)
            y_ws = layer.forward(x, channels=(b, e))
            torch.cuda.synchronize()
            assert torch.equal(y_static, y_ws), (case, m, (b, e))
        layer.close()
