"""GPU: the one-row FFN with pair units in the gate_up GEMV against the same layer run as separate calls.

With a spill for the pairs it may split, the one-row gate_up deals its (strip pair, K half) units evenly over the
CUs, ceil(2 pairs / CUs) waves per workgroup. Where that count is odd, one pair per two workgroups has its halves
in both; it leaves its act columns to the down GEMV, which forms them from the halves' fp32 sums while staging.
hm_ffn_forward and hm_ffn_block_forward take this path at one row (odd counts only where the down GEMV has one
strip group per workgroup); hm_ffn_gate_up and hm_ffn_down (act handed to the caller) do not. Both plans give
each pair two waves over the same K halves (hidden 2048..8191), so the outputs agree bit for bit; the float64
oracle checks the layer as well."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu

_CACHE = {}


def _layer(oracle, hm, device, hidden, inter, group, dtype, seed, f64=False):
    key = (hidden, inter, group, dtype, seed, f64)
    if key not in _CACHE:
        _CACHE.clear()
        rng = np.random.default_rng(seed)
        ws = [oracle.random_weights(rng, k, n, group, dtype) for k, n in ((hidden, inter), (hidden, inter), (inter, hidden))]
        layer = hm.FfnLayer.from_logical(*(logical_to_device(w, dtype, device) for w in ws), group, dtype=TORCH[dtype])
        wf = tuple(oracle.weights_f64(*w, group, dtype) for w in ws) if f64 else None
        _CACHE[key] = (layer, wf)
    return _CACHE[key]


def _units(inter_channels):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return -(-2 * (inter_channels // 16) // cus)


@pytest.mark.parametrize("hidden,inter,group,dtype,channels", [
    (4096, 9216, 128, "fp16", None),              # 5 units per workgroup, a partial last workgroup
    (4096, 14336, 128, "bf16", None),             # 7 (the Llama-3-8B layer)
    (4096, 12288, 64, "fp16", None),              # 6: even, no pair split
    (4096, 17408, 32, "fp16", None),              # 9, groups of 32
    (4096, 14336, 128, "fp16", (2048, 11264)),    # a channel range of 9216: 5
    (5120, 13824, 64, "bf16", None),              # Qwen2.5-14B: 7 (whole pairs kept: two down strip groups)
    (4096, 21504, 128, "fp16", None),             # 11
    (4096, 25600, 64, "bf16", None),              # 13
    (4096, 29696, 128, "fp16", None),             # 15: down waves forming 16 pairs (256 columns)
    (3968, 9216, 128, "fp16", None),              # 5, 31 K tiles: halves of 16 and 15
    (3968, 14336, 32, "bf16", None),              # 7, 31 K tiles, groups of 32
    (6144, 14336, 32, "bf16", None),              # 7, but two down strip groups per workgroup: whole pairs
])
def test_forward_equals_separate_calls(oracle, hm, device, hidden, inter, group, dtype, channels):
    layer, _ = _layer(oracle, hm, device, hidden, inter, group, dtype, 31)
    b, e = (0, inter) if channels is None else channels
    print(f"units {_units(e - b)} hidden {hidden} channels [{b}, {e})", flush=True)
    rng = np.random.default_rng(hidden + e)
    for rep in range(2):  # the second call finds the first call's spill and act in the workspace
        _, x = make_x(oracle, rng, 1, hidden, dtype, device)
        y = layer.forward(x, channels=(b, e))
        ref = layer.down(layer.gate_up(x, channels=(b, e)), channels=(b, e))
        torch.cuda.synchronize()
        assert torch.equal(y, ref), (hidden, inter, group, dtype, channels, rep)
    # then a narrower range on the same workspace: its own pairs only
    narrow = (b, min(e, b + 9216))
    _, x = make_x(oracle, rng, 1, hidden, dtype, device)
    y = layer.forward(x, channels=narrow)
    ref = layer.down(layer.gate_up(x, channels=narrow), channels=narrow)
    torch.cuda.synchronize()
    assert torch.equal(y, ref), narrow


@pytest.mark.parametrize("hidden,inter,group,dtype", [
    (2048, 8192, 128, "fp16"),   # Llama-3.2-1B: 4 units per workgroup, no pair split
    (2048, 9216, 64, "bf16"),    # 5 units, halves of 8 tiles
    (4096, 9216, 128, "fp16"),   # 5 units
])
def test_forward_against_oracle(oracle, hm, device, hidden, inter, group, dtype):
    layer, wf = _layer(oracle, hm, device, hidden, inter, group, dtype, 37, f64=True)
    print(f"units {_units(inter)} hidden {hidden} inter {inter}", flush=True)
    rng = np.random.default_rng(41 + inter)
    x64, x = make_x(oracle, rng, 1, hidden, dtype, device)
    y = layer.forward(x)
    torch.cuda.synchronize()
    wg, wu, wd = wf
    act = oracle.silu(x64 @ wg) * (x64 @ wu)
    act = oracle.round_to(act.astype(np.float32), dtype).astype(np.float64)
    assert_close(oracle, host_f64(y), act @ wd, dtype, f"one-row FFN [{hidden}x{inter}] g={group} {dtype}")


@pytest.mark.parametrize("dtype,inter", [("fp16", 14336), ("bf16", 9216)])
def test_block_forward_equals_separate_calls(oracle, hm, device, dtype, inter):
    # x += down(SwiGLU(RMSNorm(x) * w W_gate_up)): the gate_up stages the norm, the down GEMV forms the split pairs
    # and adds into x; against rmsnorm, gate_up, down and residual_add2 as separate calls.
    hidden = 4096
    layer, _ = _layer(oracle, hm, device, hidden, inter, 128, dtype, 43)
    print(f"units {_units(inter)} block forward {dtype}", flush=True)
    rng = np.random.default_rng(47)
    _, x = make_x(oracle, rng, 1, hidden, dtype, device)
    w = torch.from_numpy(rng.uniform(0.5, 1.5, hidden).astype(np.float32)).to(device).to(TORCH[dtype])
    normed = torch.empty_like(x)
    hm.rmsnorm(normed, x, w, 1e-5)
    ref = x.clone()
    hm.residual_add2(ref, layer.down(layer.gate_up(normed)))
    got = x.clone()
    layer.block_forward(got, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
