"""CPU: checkpoint ingestion. GPTQ nibble unpacking (the library against the oracle, the oracle against a
hand-built word and against the published GPTQ packing run forwards), and the pre-saved cache writer (padding
alignment rules, padded tiles, K-split files against the reference's tile-mask split)."""

import json
import os

import numpy as np
import pytest


def _gptq_pack(q):
    """The GPTQ checkpoint packing: word (r, o) = sum_i q[8 r + i, o] << 4 i (the published int32 layout of
    GPTQ qweight, In/8 rows)."""
    k, n = q.shape
    w = np.zeros((k // 8, n), np.uint32)
    for i in range(8):
        w |= q[i::8].astype(np.uint32) << np.uint32(4 * i)
    return w.view(np.int32)


def test_gptq_unpack_known_answer(oracle):
    packed = np.array([[0x76543210, 0xFEDCBA98]], np.uint32).view(np.int32)
    got = oracle.gptq_unpack(packed)
    assert got.shape == (8, 2)
    np.testing.assert_array_equal(got[:, 0], np.arange(8))
    np.testing.assert_array_equal(got[:, 1], np.arange(8, 16))


def test_gptq_unpack_inverts_gptq_packing(oracle):
    rng = np.random.default_rng(11)
    q = rng.integers(0, 16, (256, 48), dtype=np.uint8)
    np.testing.assert_array_equal(oracle.gptq_unpack(_gptq_pack(q)), q)


def test_gptq_zeros_known_answer(oracle):
    packed = np.array([[0x76543210, 0xFEDCBA98]], np.uint32).view(np.int32)
    np.testing.assert_array_equal(oracle.gptq_unpack_zeros(packed, add_one=False)[0], np.arange(16))
    np.testing.assert_array_equal(oracle.gptq_unpack_zeros(packed)[0], np.arange(1, 17))


def test_gptq_library_matches_oracle(hm, oracle):
    rng = np.random.default_rng(12)
    qw = rng.integers(-2 ** 31, 2 ** 31, (16, 40), dtype=np.int64).astype(np.int32)
    np.testing.assert_array_equal(hm.gptq_unpack_qweight(qw), oracle.gptq_unpack(qw))
    qz = rng.integers(-2 ** 31, 2 ** 31, (6, 5), dtype=np.int64).astype(np.int32)
    np.testing.assert_array_equal(hm.gptq_unpack_qzeros(qz), oracle.gptq_unpack_zeros(qz))
    np.testing.assert_array_equal(hm.gptq_unpack_qzeros(qz, add_one=False), oracle.gptq_unpack_zeros(qz, add_one=False))
    with pytest.raises(ValueError):
        hm.gptq_unpack_qweight(np.zeros(8, np.int32))


# ---- pre-saved cache ------------------------------------------------------------------------------------

def test_pad_alignment_rules(hm):
    from heteromega_amd import presaved as ps
    assert ps.pad_alignment(False) == (0, 0)
    assert ps.pad_alignment(True) == (2048, 2048)
    assert ps.pad_alignment(1024) == (1024, 1024)
    assert ps.pad_alignment(0) == (0, 0)
    assert ps.pad_alignment([256, 0]) == (256, 0)
    assert ps.pad_alignment([0, 0], {"gate": [512, 512]}, "gate") == (0, 0)   # overrides apply only when on
    assert ps.pad_alignment(True, {"down": [0, 1024]}, "down") == (0, 1024)
    assert ps.pad_alignment(True, {"down": [0, 1024]}, "up") == (2048, 2048)
    assert ps.packed_extent(5120, 13824, (2048, 2048)) == (6144, 14336)
    assert ps.packed_extent(4096, 14336, (2048, 2048)) == (4096, 14336)


def _layer(oracle, rng, hidden, inter):
    return {name: oracle.random_weights(rng, *shape, 128, "bf16", 0.002, 0.02, 0, 16)
            for name, shape in (("gate", (hidden, inter)), ("up", (hidden, inter)), ("down", (inter, hidden)))}


def test_padded_tiles_hold_the_block_and_zeros(hm, oracle, tmp_path):
    from heteromega_amd import presaved as ps
    rng = np.random.default_rng(13)
    hidden, inter = 256, 640
    layer = _layer(oracle, rng, hidden, inter)
    m = ps.write_presaved(str(tmp_path), [layer], hidden, inter, pad_packed=1024)
    assert m["pad_packed_weights"] == 1024 and m["split_k_by_layer"] == {}
    for name, (k, n) in (("gate", (hidden, inter)), ("down", (inter, hidden))):
        raw = np.fromfile(ps.packed_path(str(tmp_path), 0, name), np.uint8)
        q, s, z = layer[name]
        q2, s2, z2 = oracle.unpack_tiles(raw, 1024, 1024)
        np.testing.assert_array_equal(q2[:k, :n], q)
        np.testing.assert_array_equal(s2[:k // 128, :n], s)
        np.testing.assert_array_equal(z2[:k // 128, :n], z)
        assert not q2[k:].any() and not q2[:, n:].any() and not s2[k // 128:].any() and not z2[:, n:].any()


def test_split_files_are_the_reference_tile_mask_split(hm, oracle, tmp_path):
    # _split_packed_bin_from_file (llama3_8b_w4a16_model.py:468-530) keeps, in file order, the tiles whose tile
    # row is below K0/128 (packed0) and the rest (packed1); writing the two row blocks packed on their own
    # (:1105-1140) must give the same two files.
    from heteromega_amd import presaved as ps
    rng = np.random.default_rng(14)
    hidden, inter = 384, 640
    layer = _layer(oracle, rng, hidden, inter)
    whole, split = tmp_path / "whole", tmp_path / "split"
    ps.write_presaved(str(whole), [layer], hidden, inter)
    ps.write_presaved(str(split), [layer], hidden, inter, split_k_by_layer={"gate": 256, "down": 384})
    for name, k, n, k0 in (("gate", hidden, inter, 256), ("down", inter, hidden, 384)):
        full = np.fromfile(ps.packed_path(str(whole), 0, name), np.uint8).reshape(-1, 4352)
        tk, tn = k // 128, n // 64
        row_of = np.empty(tk * tn, np.int64)
        for c in range(tn):
            for r in range(tk):
                row_of[oracle.tile_index(c, r, tk, tn)] = r
        mask0 = row_of < k0 // 128
        p0, p1 = ps.split_paths(str(split), 0, name, k0)
        np.testing.assert_array_equal(np.fromfile(p0, np.uint8).reshape(-1, 4352), full[mask0])
        np.testing.assert_array_equal(np.fromfile(p1, np.uint8).reshape(-1, 4352), full[~mask0])
    assert os.path.exists(ps.packed_path(str(split), 0, "up"))
    with open(split / "manifest.json") as f:
        man = json.load(f)
    assert man["split_k_by_layer"] == {"gate": 256, "down": 384}
    # the keys the reference's manifest check compares (llama3_8b_w4a16_model.py:962-976) that concern the MLP
    for key in ("format_version", "use_packed_weights", "pad_packed_weights", "split_k_by_layer", "num_hidden_layers",
                "hidden_size", "intermediate_size", "groupsize"):
        assert key in man


def test_unpacked_layout_files(hm, oracle, tmp_path):
    # out_groups_v2: qweight [N, K/2] with the even k in the low nibble, scales and zeros [N, K/group].
    from heteromega_amd import presaved as ps
    rng = np.random.default_rng(15)
    layer = _layer(oracle, rng, 256, 384)
    ps.write_presaved(str(tmp_path), [layer], 256, 384, use_packed=False)
    q, s, z = layer["gate"]
    raw = np.fromfile(tmp_path / "layer_0_gate.qweight.bin", np.uint8).reshape(384, 128)
    np.testing.assert_array_equal(raw[5, 7] & 0xF, q[14, 5])
    np.testing.assert_array_equal(raw[5, 7] >> 4, q[15, 5])
    np.testing.assert_array_equal(np.fromfile(tmp_path / "layer_0_gate.scales.bin", np.uint16).reshape(384, 2), s.T)
    np.testing.assert_array_equal(np.fromfile(tmp_path / "layer_0_gate.zeros.bin", np.uint8).reshape(384, 2), z.T)
    with open(tmp_path / "manifest.json") as f:
        assert json.load(f)["unpacked_layout"] == "out_groups_v2"
