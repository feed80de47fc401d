"""Pre-saved weight cache: the directory of raw `.bin` files and `manifest.json` the reference's model loader
writes once and reads on every start (_prepare_presaved_weights, llama3_8b_w4a16_model.py:931-1169;
qwen25_14b_w4a16_model.py:1213-1520), restricted to the MLP matrices this engine computes.

Files, per layer i and matrix name in ("gate", "up", "down"):
  use_packed_weights true:
    layer_{i}_{name}.packed.bin                       the [K, N] matrix in 4352-byte tiles, padded per the manifest
    layer_{i}_{name}.k{s}.packed0.bin / .packed1.bin  when split_k_by_layer[name] = s: rows [0, s) and [s, K),
                                                      each packed (and padded) on its own (:1105-1140)
  use_packed_weights false ("unpacked_layout": "out_groups_v2", :1158-1164):
    layer_{i}_{name}.qweight.bin  [N, K/2] u8, low nibble = even k
    layer_{i}_{name}.scales.bin   [N, K/group] bf16
    layer_{i}_{name}.zeros.bin    [N, K/group] int8
Padding (padPackedWeights, :546-608; per-matrix pairs in qwen25_14b_w4a16_model.py:104-217): K and N are rounded
up to the alignment with zero weights, zero scales and zero zero-points; the engine keeps the leading [K, N]
block, so the padding costs nothing at run time.
"""
import json
import os

import numpy as np
import torch

from . import ffn as _ffn

MLP_MATRICES = ("gate", "up", "down")
LEGACY_PAD_ALIGNMENT = 2048  # padPackedWeights: true (qwen25_14b_w4a16_model.py:93)


def _round_up(v, m):
    return v if m <= 0 else (v + m - 1) // m * m


def _pad_pair(value):
    if isinstance(value, (list, tuple)) and len(value) >= 2:
        out = []
        for v in value[:2]:
            try:
                v = int(v)
            except (TypeError, ValueError):
                v = 0
            out.append(v if v > 0 else 0)
        return tuple(out)
    return (0, 0)


def pad_alignment(pad_packed, pad_by_layer=None, name=""):
    """(align_k, align_n) of one matrix: `pad_packed` is false/true (2048)/an integer/a [k, n] pair, and a
    per-name pair in pad_by_layer overrides it when padding is on (_resolve_layer_pad_packed_alignment,
    qwen25_14b_w4a16_model.py:197-217)."""
    if isinstance(pad_packed, (list, tuple)):
        enabled = _pad_pair(pad_packed)
        if enabled == (0, 0):
            return (0, 0)
    else:
        if isinstance(pad_packed, bool):
            align = LEGACY_PAD_ALIGNMENT if pad_packed else 0
        else:
            try:
                align = int(pad_packed or 0)
            except (TypeError, ValueError):
                align = 0
        if align <= 0:
            return (0, 0)
        enabled = (align, align)
    if isinstance(pad_by_layer, dict) and name in pad_by_layer:
        return _pad_pair(pad_by_layer[name])
    return enabled


def packed_extent(k, n, align):
    """Packed [K, N] of a logical [k, n] matrix under alignment (align_k, align_n)."""
    return _round_up(k, align[0]), _round_up(n, align[1])


def matrix_shape(name, hidden, inter):
    return (inter, hidden) if name == "down" else (hidden, inter)


def packed_path(directory, layer, name):
    return os.path.join(directory, f"layer_{layer}_{name}.packed.bin")


def split_paths(directory, layer, name, split_k):
    """(_split_packed_paths, llama3_8b_w4a16_model.py:460-465)."""
    tag = f"k{int(split_k)}"
    return (os.path.join(directory, f"layer_{layer}_{name}.{tag}.packed0.bin"),
            os.path.join(directory, f"layer_{layer}_{name}.{tag}.packed1.bin"))


# ---- writer (the reference's preprocessing step, for tests and for converting checkpoints) --------------

def pack_padded(q, scales, zeros, align):
    """Tiles of [K, N] q (u8), scales [K/128, N] (bf16 bits), zeros [K/128, N], zero-padded to the alignment
    (_pack_weights_packed, llama3_8b_w4a16_model.py:546-608, for group 128)."""
    q = _ffn._host_array(q, np.uint8)
    s = _ffn._host_array(scales, np.uint16)
    z = _ffn._host_array(zeros, np.int8)
    k, n = q.shape
    kp, np_ = packed_extent(k, n, align)
    if (kp, np_) != (k, n):
        q = np.pad(q, ((0, kp - k), (0, np_ - n)))
        s = np.pad(s, ((0, kp // _ffn.kTileK - s.shape[0]), (0, np_ - n)))
        z = np.pad(z, ((0, kp // _ffn.kTileK - z.shape[0]), (0, np_ - n)))
    return _ffn.pack_w4a16(q, s, z)


def write_presaved(directory, layers, hidden, inter, pad_packed=False, split_k_by_layer=None, pad_by_layer=None,
                   use_packed=True, model_name="model", extra_manifest=None):
    """Writes the MLP part of a pre-saved cache. layers: a list of {"gate"|"up"|"down": (q [K, N] u8,
    scales [K/128, N] bf16 bits, zeros [K/128, N] int)} on the host, group 128."""
    os.makedirs(directory, exist_ok=True)
    split_k_by_layer = dict(split_k_by_layer or {}) if use_packed else {}
    group = _ffn.kTileK
    for i, layer in enumerate(layers):
        for name in MLP_MATRICES:
            q, s, z = layer[name]
            q, s, z = _ffn._host_array(q, np.uint8), _ffn._host_array(s, np.uint16), _ffn._host_array(z, np.int8)
            k, n = matrix_shape(name, hidden, inter)
            if q.shape != (k, n):
                raise ValueError(f"write_presaved: layer {i} {name} is {q.shape}, expected {(k, n)}")
            if not use_packed:
                group = k // s.shape[0]
                q_out_in = q.T.astype(np.uint8)
                packed = (q_out_in[:, 0::2] & 0xF) | ((q_out_in[:, 1::2] & 0xF) << 4)
                base = os.path.join(directory, f"layer_{i}_{name}")
                np.ascontiguousarray(packed.astype(np.uint8)).tofile(base + ".qweight.bin")
                np.ascontiguousarray(s.T).tofile(base + ".scales.bin")
                np.ascontiguousarray(z.T).tofile(base + ".zeros.bin")
                continue
            if s.shape[0] * _ffn.kTileK != k:
                raise ValueError("write_presaved: packed tiles hold group 128")
            align = pad_alignment(pad_packed, pad_by_layer, name)
            split = int(split_k_by_layer.get(name, 0))
            if 0 < split < k:
                g0 = split // _ffn.kTileK
                p0, p1 = split_paths(directory, i, name, split)
                pack_padded(q[:split], s[:g0], z[:g0], align).tofile(p0)
                pack_padded(q[split:], s[g0:], z[g0:], align).tofile(p1)
            else:
                pack_padded(q, s, z, align).tofile(packed_path(directory, i, name))
    manifest = {
        "format_version": 1,
        "model_name": model_name,
        "use_packed_weights": bool(use_packed),
        "pad_packed_weights": pad_packed,
        "split_k_by_layer": split_k_by_layer,
        "num_hidden_layers": len(layers),
        "hidden_size": hidden,
        "intermediate_size": inter,
        "groupsize": group,
    }
    if pad_by_layer:
        manifest["pad_packed_weights_by_layer"] = {k: list(v) for k, v in sorted(pad_by_layer.items())}
    if not use_packed:
        manifest["unpacked_layout"] = "out_groups_v2"
    if extra_manifest:
        manifest.update(extra_manifest)
    with open(os.path.join(directory, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)
    return manifest


# ---- reader ---------------------------------------------------------------------------------------------

def read_manifest(directory):
    path = os.path.join(directory, "manifest.json")
    with open(path) as f:
        m = json.load(f)
    for key in ("hidden_size", "intermediate_size", "num_hidden_layers"):
        if key not in m:
            raise ValueError(f"{path}: no '{key}'")
    return m


def _read(path, nbytes):
    if not os.path.exists(path):
        raise FileNotFoundError(f"pre-saved weights: missing {path}")
    size = os.path.getsize(path)
    if size != nbytes:
        raise ValueError(f"pre-saved weights: {path} has {size} bytes, expected {nbytes}")
    return torch.from_numpy(np.fromfile(path, dtype=np.uint8))


def _tiles_on_device(path, k, n, device):
    nbytes = _ffn.packed_bytes(k, n)
    if nbytes < 0:
        raise ValueError(f"pre-saved weights: packed extent [{k}, {n}] is not a multiple of 128 x 64")
    return _read(path, nbytes).to(device)


def _logical_from_tiles(path, k, n, align, dtype, device, stream):
    kp, np_ = packed_extent(k, n, align)
    w = _ffn.RepackedMatrix.from_tiles(_tiles_on_device(path, kp, np_, device), kp, np_, k, n, dtype, stream)
    try:
        out = w.to_logical(stream)
        torch.cuda.synchronize(device)
        return out
    finally:
        w.close()


def _logical_matrix(directory, manifest, layer, name, dtype, device, stream):
    """(q [K, N] u8, scales [K/128, N] dtype, zeros [K/128, N] u8) of one matrix, on the device."""
    k, n = matrix_shape(name, manifest["hidden_size"], manifest["intermediate_size"])
    if not manifest.get("use_packed_weights", True):
        if manifest.get("unpacked_layout", "out_groups_v2") != "out_groups_v2":
            raise ValueError(f"pre-saved weights: unknown unpacked_layout {manifest.get('unpacked_layout')!r}")
        base = os.path.join(directory, f"layer_{layer}_{name}")
        # the group count comes from the scales file's size (helper.cpp:1091-1097)
        groups = os.path.getsize(base + ".scales.bin") // 2 // n if os.path.exists(base + ".scales.bin") else 0
        if groups <= 0 or k % groups:
            raise ValueError(f"pre-saved weights: {base}.scales.bin does not hold [{n}, K/group] bf16 scales")
        group = k // groups
        packed = _read(base + ".qweight.bin", n * k // 2).to(device).view(n, k // 2)
        q = torch.stack((packed & 0xF, packed >> 4), dim=2).view(n, k).t().contiguous()
        s = _read(base + ".scales.bin", n * (k // group) * 2).view(torch.bfloat16).to(device).view(n, k // group)
        z = _read(base + ".zeros.bin", n * (k // group)).to(device).view(n, k // group)
        return q, s.t().contiguous().to(dtype), z.t().contiguous(), group
    group = _ffn.kTileK  # a tile holds one scale and zero per column (the packer keeps group 128 of finer ones)
    align = pad_alignment(manifest.get("pad_packed_weights", False), manifest.get("pad_packed_weights_by_layer"), name)
    split = int(manifest.get("split_k_by_layer", {}).get(name, 0))
    if 0 < split < k:
        if split % _ffn.kTileK:
            raise ValueError(f"pre-saved weights: split_k {split} of {name} is not a multiple of 128")
        p0, p1 = split_paths(directory, layer, name, split)
        if not (os.path.exists(p0) and os.path.exists(p1)):  # untagged names of older caches (helper.cpp:1064-1068)
            p0, p1 = (os.path.join(directory, f"layer_{layer}_{name}.packed{j}.bin") for j in (0, 1))
        a = _logical_from_tiles(p0, split, n, align, dtype, device, stream)
        b = _logical_from_tiles(p1, k - split, n, align, dtype, device, stream)
        return tuple(torch.cat((x, y), dim=0) for x, y in zip(a, b)) + (group,)
    return _logical_from_tiles(packed_path(directory, layer, name), k, n, align, dtype, device, stream) + (group,)


def load_ffn_layer(directory, layer, manifest=None, dtype=torch.bfloat16, device="cuda", stream=None):
    """FfnLayer of one layer of a pre-saved cache. Unsplit packed matrices with one padding for all three
    go straight from the tiles to the strip layout; split, unpacked or unevenly padded ones pass through the
    logical form on the device."""
    m = read_manifest(directory) if manifest is None else manifest
    if not 0 <= layer < int(m["num_hidden_layers"]):
        raise ValueError(f"pre-saved weights: no layer {layer} in {directory}")
    hidden, inter = int(m["hidden_size"]), int(m["intermediate_size"])
    device = torch.device(device)
    if m.get("use_packed_weights", True):
        splits = m.get("split_k_by_layer", {}) or {}
        aligns = [pad_alignment(m.get("pad_packed_weights", False), m.get("pad_packed_weights_by_layer"), n) for n in MLP_MATRICES]
        ph, pi = packed_extent(hidden, inter, aligns[0])
        even = aligns[1] == aligns[0] and packed_extent(inter, hidden, aligns[2]) == (pi, ph)
        if even and not any(0 < int(splits.get(n, 0)) < matrix_shape(n, hidden, inter)[0] for n in MLP_MATRICES):
            gate = _tiles_on_device(packed_path(directory, layer, "gate"), ph, pi, device)
            up = _tiles_on_device(packed_path(directory, layer, "up"), ph, pi, device)
            down = _tiles_on_device(packed_path(directory, layer, "down"), pi, ph, device)
            f = _ffn.FfnLayer.from_tiles(gate, up, down, hidden, inter, dtype, stream, packed_hidden=ph, packed_inter=pi)
            torch.cuda.synchronize(device)  # the staged tiles are freed on return; loading is a one-time step
            return f
    mats = [_logical_matrix(directory, m, layer, n, dtype, device, stream) for n in MLP_MATRICES]
    if len({x[3] for x in mats}) != 1:
        raise ValueError(f"pre-saved weights: layer {layer} mixes group sizes {[x[3] for x in mats]}")
    f = _ffn.FfnLayer.from_logical(*(x[:3] for x in mats), mats[0][3], dtype, stream)
    torch.cuda.synchronize(device)
    return f


def load_presaved(directory, dtype=torch.bfloat16, device="cuda", stream=None, num_layers=None):
    """GpuFfnModel holding the MLP of every layer (or the first num_layers) of a pre-saved cache
    (load_quantized_weights_from_bins, llama3_8b_w4a16_model.py:905, for the FFN part)."""
    m = read_manifest(directory)
    n = int(m["num_hidden_layers"]) if num_layers is None else int(num_layers)
    model = _ffn.GpuFfnModel(dtype)
    for i in range(n):
        model.append(load_ffn_layer(directory, i, m, dtype, device, stream))
    return model


__all__ = ["MLP_MATRICES", "LEGACY_PAD_ALIGNMENT", "pad_alignment", "packed_extent", "packed_path", "split_paths",
           "pack_padded", "write_presaved", "read_manifest", "load_ffn_layer", "load_presaved"]
