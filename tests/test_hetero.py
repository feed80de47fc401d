"""CPU: the hetero split descriptors (include/hm_w4a16.h split section; heteromega_amd/hetero.py).

Known answers of the split-type rule (npuSetup.cpp:1283-1291) and of get_layer_id (npuSetup.cpp:635-653), the
config table's loader rules and exact-key lookup (npuSetup.cpp:1312-1319, :1467, :1763; hetero_compute.cpp:98-106),
and rejections modelled on tests/ffn_deploy/contract_test.cpp for the merged-FFN contract's shape, partition and
buffer sizes (include/heteromega/merged_ffn_contract.hpp)."""

import pytest


@pytest.fixture(scope="module")
def het(hm):
    return hm.hetero


@pytest.mark.parametrize("shape,expected", [
    ((512, 4096, 14336, 512, 2048, 14336), 2048),   # K differs: K split at npuK
    ((512, 4096, 14336, 256, 1024, 7168), 1024),    # K differs with M and N: the K split takes precedence
    ((2048, 4096, 14336, 512, 4096, 14336), -1),    # only M differs: M split
    ((512, 4096, 14336, 512, 4096, 7168), -2),      # N differs: N split
    ((2048, 4096, 14336, 512, 4096, 7168), -2),     # M and N differ: N split (M split needs N equal)
    ((512, 4096, 14336, 512, 4096, 14336), -1),     # nothing differs: the loader's default
])
def test_split_type_rule(het, shape, expected):
    assert het.split_type(*shape) == expected


def test_layer_ids(het):
    for name, lid in (("qkv", 8), ("q", 1), ("k", 2), ("v", 3), ("o", 4), ("gate", 5), ("up", 6), ("down", 7), ("", 0), ("mlp", 0)):
        assert het.get_layer_id(name) == lid, name


def test_config_map_entries_and_exact_lookup(het):
    cm = het.ConfigMap()
    assert cm.add_gemm(512, 4096, 14336, "gate", 512, 4096, 14336, config=3)  # a whole-M entry: M split by default
    assert cm.add_gemm(512, 14336, 4096, "down", 512, 7168, 4096, chunk_id=2)  # a K split, for chunk 2 only
    assert not cm.add_gemm(512, 4096, 4096, "q", 0, 4096, 4096)  # npuM == 0: GPU-only, skipped by the loader
    cm.add_gemv(4096, 14336, "up", npuN=4096, cpuN=1024, cpuThreads=8)
    assert len(cm) == 3
    g = cm.find(512, 4096, 14336, "gate")
    assert (g.hw_idx, g.inst_idx, g.npuM, g.npuK, g.npuN, g.cpuN, g.cpuThreads, g.config, g.split_type) == (-1, -1, 512, 4096, 14336, 0, 1, 3, -1)
    d = cm.find(512, 14336, 4096, "down", chunk_id=2)
    assert d.split_type == 7168
    assert cm.find(512, 14336, 4096, "down") is None  # chunk -1 is not a wildcard
    assert cm.find(512, 14336, 4096, "down", chunk_id=3) is None
    assert cm.find(512, 4096, 4096, "q") is None
    u = cm.find(1, 4096, 14336, 6)
    assert (u.npuM, u.npuK, u.npuN, u.cpuN, u.cpuThreads, u.split_type) == (1, 4096, 4096, 1024, 8, 0)
    cm.add_gemv(4096, 14336, "up", npuN=0, cpuN=2048)  # a later entry for the same key replaces the first
    assert cm.find(1, 4096, 14336, "up").cpuN == 2048 and len(cm) == 3


@pytest.mark.parametrize("args", [
    (512, 4096, 14336, "gate", 512, 8192, 14336),   # npuK beyond forK
    (512, 4096, 14336, "gate", 512, 1000, 14336),   # K shares not multiples of 128
    (512, 4096, 14336, "gate", -1, 4096, 14336),    # negative share
    (0, 4096, 14336, "gate", 512, 4096, 14336),     # empty projection
    (512, 4096, 14336, "gate", 512, 0, 14336),
])
def test_config_map_rejects_bad_entries(het, args):
    cm = het.ConfigMap()
    with pytest.raises(ValueError):
        cm.add_gemm(*args)
    assert len(cm) == 0


def test_merged_ffn_contract_sizes_and_support(het, hm):
    # tests/ffn_deploy/contract_test.cpp:52-58: m 512, H 4096, I 14336, P 6400 -> 4,194,304 / 6,553,600 / 31,195,136 bytes
    assert het.merged_ffn_check(512, 4096, 14336, 6400) == (4194304, 6553600, 31195136)
    lib = hm._lib.load()
    assert lib.hm_merged_ffn_supports(512, 4096, 14336, 512, 4096, 14336)
    for rows, h, inter in ((1, 4096, 14336), (256, 4096, 14336), (512, 4096, 11008)):
        assert not lib.hm_merged_ffn_supports(512, 4096, 14336, rows, h, inter)


@pytest.mark.parametrize("m,h,inter,p", [
    (0, 4096, 14336, 6400), (-128, 4096, 14336, 6400), (513, 4096, 14336, 6400),  # m (contract_test.cpp:77-80)
    (512, 4096, 14336, 0), (512, 4096, 14336, 128), (512, 4096, 14336, 6401),     # channels (:81-83)
    (512, 4096, 14336, 8448), (512, 4096, 14336, 14336),
    (512, 4096, 14000, 6400), (512, 4000, 14336, 6400),                          # shapes off the 128 grid
    (2 ** 62 // 512 * 512, 2 ** 62 // 128 * 128, 14336, 6400),                   # overflowing sizes (:89-91)
])
def test_merged_ffn_contract_rejections(het, m, h, inter, p):
    with pytest.raises(ValueError):
        het.merged_ffn_check(m, h, inter, p)
