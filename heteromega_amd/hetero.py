"""Host mirror of the reference's hetero split descriptors over the C ABI (include/hm_w4a16.h, split section).

The reference keys each projection's kernel config by NPUKey {forM, forK, forN, layer_id, chunk_id} and stores an
NPUValue {hw_idx, inst_idx, npuM, npuK, npuN, cpuN, cpuThreads, config, split_type}
(include/unified_llm_w4a16_hetero/npuSetup.hpp:93-114). ConfigMap restates that table and its loader's rules
(npuSetup.cpp:1283-1319, :1467, :1763); hetero_linear runs the split an entry describes with every share on the
GPU (hetero_compute.cpp:189-259, 282-447, 497-560, 633-805).
"""

import ctypes

import torch

from . import _lib
from .ffn import _call, _aligned, _ptr, _stream, _workspace


class NPUValue(ctypes.Structure):
    """hm_split_desc: the config entry of one projection."""

    _fields_ = [(name, ctypes.c_int32) for name in ("hw_idx", "inst_idx", "npuM", "npuK", "npuN", "cpuN", "cpuThreads", "config", "split_type")]

    def __repr__(self):
        return "NPUValue(" + ", ".join(f"{n}={getattr(self, n)}" for n, _ in self._fields_) + ")"


def get_layer_id(layer_type):
    """qkv 8, q 1, k 2, v 3, o 4, gate 5, up 6, down 7, else 0 (npuSetup.cpp:635-653)."""
    return _lib.load().hm_layer_id(layer_type.encode() if isinstance(layer_type, str) else layer_type)


def split_type(forM, forK, forN, npuM, npuK, npuN):
    """npuK for a K split (precedence), -1 for an M split, -2 for an N split (npuSetup.cpp:1283-1291)."""
    return _lib.load().hm_split_type(forM, forK, forN, npuM, npuK, npuN)


class ConfigMap:
    """config_map: entries keyed by (M, K, N, layer_id, chunk_id), looked up by exact key (hetero_compute.cpp:98-106)."""

    def __init__(self):
        h = ctypes.c_void_p()
        _call(_lib.load().hm_split_table_create(ctypes.byref(h)))
        self._h = h

    def add_gemm(self, forM, forK, forN, layer, npuM, npuK, npuN, config=-1, chunk_id=-1):
        """A GEMM kernel entry; returns False when the reference would skip it (npuM == 0: GPU-only)."""
        stored = ctypes.c_int32()
        lid = layer if isinstance(layer, int) else get_layer_id(layer)
        _call(_lib.load().hm_split_table_add_gemm(self._h, forM, forK, forN, lid, chunk_id, npuM, npuK, npuN, config, ctypes.byref(stored)))
        return bool(stored.value)

    def add_gemv(self, forK, forN, layer, npuN=0, cpuN=0, cpuThreads=1, config=-1, chunk_id=-1):
        lid = layer if isinstance(layer, int) else get_layer_id(layer)
        _call(_lib.load().hm_split_table_add_gemv(self._h, forK, forN, lid, chunk_id, npuN, cpuN, cpuThreads, config))

    def find(self, M, K, N, layer, chunk_id=-1):
        """The entry for this exact key, or None."""
        v = NPUValue()
        lid = layer if isinstance(layer, int) else get_layer_id(layer)
        st = _lib.load().hm_split_table_find(self._h, M, K, N, lid, chunk_id, ctypes.byref(v))
        return v if st == _lib.HM_OK else None

    def __len__(self):
        return _lib.load().hm_split_table_size(self._h)

    def close(self):
        if self._h:
            _lib.load().hm_split_table_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def hetero_linear(out, x, value, w0, w1=None, k=None, stream=None):
    """out [M, N] = x [M, K] @ W split as `value` (an NPUValue or None) describes, every share on the GPU. A K split
    needs the second share's matrix w1 (rows [K0, K) of W, K0 = value.split_type)."""
    k_split = value is not None and value.split_type > 0
    if k is None:
        k = value.split_type + w1.k if k_split and w1 is not None else w0.k
    m, n = x.size(0), out.size(1)
    lib = _lib.load()
    vp = ctypes.byref(value) if value is not None else None
    h1 = w1._h if w1 is not None else None
    need = lib.hm_linear_split_workspace_bytes(vp, w0._h, h1, m, k, n)
    ws = _workspace(need, x.device)
    wp, wb = _aligned(ws, need)
    _call(lib.hm_linear_split(vp, w0._h, h1, _ptr(out), out.stride(0), _ptr(x), x.stride(0), m, k, n, wp, wb, _stream(stream, x.device)))
    return out


def merged_ffn_check(m, hidden, intermediate, npu_channels):
    """MergedFfnConfig's shape/partition rules and buffer sizes (merged_ffn_contract.hpp:41-127): returns
    (activation_bytes, intermediate_bytes, weight_bytes) or raises ValueError."""
    a, b, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    _call(_lib.load().hm_merged_ffn_check(m, hidden, intermediate, npu_channels, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
    return a.value, b.value, c.value


__all__ = ["NPUValue", "get_layer_id", "split_type", "ConfigMap", "hetero_linear", "merged_ffn_check"]
