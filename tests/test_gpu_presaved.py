"""GPU: loading a pre-saved weight cache (the reference's layer_{i}_{name}.packed.bin / split / unpacked files)
gives the same FFN as the same weights handed over as logical tensors, bit for bit, and matches the oracle."""

import os

import numpy as np
import pytest
import torch

from gpu_util import assert_close, host_f64, logical_to_device, make_x

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 1024, 2816


def _layers(oracle, n, seed, group=128):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        out.append({name: oracle.random_weights(rng, *shape, group, "bf16", 0.002, 0.02, 0, 16)
                    for name, shape in (("gate", (HIDDEN, INTER)), ("up", (HIDDEN, INTER)), ("down", (INTER, HIDDEN)))})
    return out


def _logical_layer(hm, layer, device, group=128):
    return hm.FfnLayer.from_logical(*(logical_to_device(layer[n], "bf16", device) for n in ("gate", "up", "down")), group,
                                    dtype=torch.bfloat16)


@pytest.mark.parametrize("case", ["plain", "pad2048", "split", "split_pad", "split_untagged", "pad_by_layer", "unpacked",
                                  "unpacked_g64"])
def test_presaved_cache_loads_bit_identical(oracle, hm, device, tmp_path, case):
    from heteromega_amd import presaved as ps
    print(f"presaved case {case}", flush=True)
    group = 64 if case == "unpacked_g64" else 128
    layers = _layers(oracle, 2, 90, group)
    kw = {
        "plain": {},
        "pad2048": {"pad_packed": True},
        "split": {"split_k_by_layer": {"gate": 512, "down": 1280}},
        "split_pad": {"pad_packed": True, "split_k_by_layer": {"up": 384, "down": 2048}},
        "split_untagged": {"split_k_by_layer": {"down": 1280}},
        "pad_by_layer": {"pad_packed": True, "pad_by_layer": {"down": [0, 1536]}},
        "unpacked": {"use_packed": False},
        "unpacked_g64": {"use_packed": False},
    }[case]
    ps.write_presaved(str(tmp_path), layers, HIDDEN, INTER, **kw)
    if case == "split_untagged":  # caches written before the split size was part of the name
        for i in range(2):
            for j, p in enumerate(ps.split_paths(str(tmp_path), i, "down", 1280)):
                os.rename(p, tmp_path / f"layer_{i}_down.packed{j}.bin")
    model = ps.load_presaved(str(tmp_path), torch.bfloat16, device)
    assert model.layers() == 2
    rng = np.random.default_rng(91)
    for m in (1, 37):
        x64, x = make_x(oracle, rng, m, HIDDEN, "bf16", device, 0.5)
        for i, layer in enumerate(layers):
            y = torch.empty((m, HIDDEN), dtype=torch.bfloat16, device=device)
            model.forward(i, x, y)
            y_ref = _logical_layer(hm, layer, device, group).forward(x)
            torch.cuda.synchronize()
            assert torch.equal(y, y_ref), (case, m, i)
    # one oracle check of the loaded model
    wf = [oracle.weights_f64(*layers[1][n], group, "bf16") for n in ("gate", "up", "down")]
    act = oracle.silu(x64 @ wf[0]) * (x64 @ wf[1])
    ref = oracle.round_to(act.astype(np.float32), "bf16").astype(np.float64) @ wf[2]
    assert_close(oracle, host_f64(y), ref, "bf16", f"pre-saved {case} M=37")


def test_presaved_rejects_truncated_file(oracle, hm, device, tmp_path):
    from heteromega_amd import presaved as ps
    layers = _layers(oracle, 1, 92)
    ps.write_presaved(str(tmp_path), layers, HIDDEN, INTER)
    path = ps.packed_path(str(tmp_path), 0, "down")
    raw = np.fromfile(path, np.uint8)
    raw[:-4352].tofile(path)
    with pytest.raises(ValueError):
        ps.load_presaved(str(tmp_path), torch.bfloat16, device)


def test_ffn_from_padded_tiles_fp16(oracle, hm, device):
    # hm_ffn_from_tiles_padded directly: gate/up packed [2048, 4096], down [4096, 2048], the layer their
    # leading [1024, 2816] blocks, activations in fp16 (bf16 scales converted once at repack).
    from heteromega_amd import presaved as ps
    layer = _layers(oracle, 1, 93)[0]
    tiles = {n: torch.from_numpy(ps.pack_padded(*layer[n], (2048, 2048))).to(device) for n in ("gate", "up", "down")}
    f = hm.FfnLayer.from_tiles(tiles["gate"], tiles["up"], tiles["down"], HIDDEN, INTER, torch.float16,
                               packed_hidden=2048, packed_inter=4096)
    ref = hm.FfnLayer.from_tiles(*(torch.from_numpy(oracle.pack_tiles(*layer[n])).to(device) for n in ("gate", "up", "down")),
                                 HIDDEN, INTER, torch.float16)
    rng = np.random.default_rng(94)
    for m in (1, 200):
        _, x = make_x(oracle, rng, m, HIDDEN, "fp16", device, 0.5)
        y, y_ref = f.forward(x), ref.forward(x)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), m
    with pytest.raises(ValueError):
        hm.FfnLayer.from_tiles(tiles["gate"], tiles["up"], tiles["down"], HIDDEN, INTER, torch.float16)
