"""ctypes binding of libhmw4a16.so (include/hm_w4a16.h).

The library is built in-tree by heteromega_amd/build.py. Loading fails loudly when it is missing: there is no
CPU fallback for any compute entry point.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhmw4a16.so")

HM_OK = 0
HM_INVALID_ARGUMENT = 1
HM_UNSUPPORTED = 2
HM_HIP_ERROR = 3
HM_OUT_OF_MEMORY = 4
HM_WORKSPACE_TOO_SMALL = 5

HM_BF16 = 0
HM_FP16 = 1

HM_GATE_UP_BLOCKED = 0
HM_GATE_UP_INTERLEAVED = 1

_STATUS_NAMES = {
    HM_INVALID_ARGUMENT: "invalid argument",
    HM_UNSUPPORTED: "unsupported",
    HM_HIP_ERROR: "HIP error",
    HM_OUT_OF_MEMORY: "out of memory",
    HM_WORKSPACE_TOO_SMALL: "workspace too small",
}


class HMError(RuntimeError):
    """A failed C ABI call: `status` is the hm_status code, the message is hm_last_error()."""

    def __init__(self, status, message):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
SZ = ctypes.c_size_t

# name: (restype, argtypes)
_SIGNATURES = {
    "hm_abi_version": (ctypes.c_int, []),
    "hm_last_error": (ctypes.c_char_p, []),
    "hm_packed_bytes": (I64, [I64, I64]),
    "hm_packed_tile_index": (I64, [I64, I64, I64, I64]),
    "hm_pack_w4a16": (ctypes.c_int, [P, P, P, I64, I64, P]),
    "hm_awq_unpack": (ctypes.c_int, [P, I64, I64, P]),
    "hm_gptq_unpack": (ctypes.c_int, [P, I64, I64, P]),
    "hm_gptq_unpack_zeros": (ctypes.c_int, [P, I64, I64, I32, P]),
    "hm_weights_from_tiles": (ctypes.c_int, [P, I64, I64, I64, I64, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_weights_from_logical": (ctypes.c_int, [P, P, P, I64, I64, I64, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_weights_from_gate_up_tiles": (ctypes.c_int, [P, I64, I64, I64, I64, I32, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_weights_dequantize": (ctypes.c_int, [P, P, I64, I32, P]),
    "hm_weights_to_logical": (ctypes.c_int, [P, P, P, P, P]),
    "hm_weights_info": (ctypes.c_int, [P, ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I32),
                                       ctypes.POINTER(I64)]),
    "hm_weights_planes": (ctypes.c_int, [P, ctypes.POINTER(P), ctypes.POINTER(I64), ctypes.POINTER(P), ctypes.POINTER(I64)]),
    "hm_weights_destroy": (ctypes.c_int, [P]),
    "hm_weights_concat": (ctypes.c_int, [ctypes.POINTER(P), ctypes.c_int32, P, ctypes.POINTER(P)]),
    "hm_linear_workspace_bytes": (SZ, [P, I64, I64, I64]),
    "hm_linear": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I64, I64, P, SZ, P]),
    "hm_linear_swiglu_workspace_bytes": (SZ, [P, I64, I64, I64]),
    "hm_linear_swiglu": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I64, I64, P, SZ, P]),
    "hm_linear_k_split_workspace_bytes": (SZ, [P, P, I64, I64, I64, I64]),
    "hm_linear_k_split": (ctypes.c_int, [P, P, P, I64, P, I64, I64, I64, I64, I64, P, SZ, P]),
    "hm_ffn_from_tiles": (ctypes.c_int, [P, P, P, I64, I64, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_ffn_from_tiles_padded": (ctypes.c_int, [P, P, P, I64, I64, I64, I64, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_ffn_from_gate_up_tiles": (ctypes.c_int, [P, P, I64, I64, I64, I32, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_ffn_from_logical": (ctypes.c_int, [P, P, P, P, P, P, P, P, P, I64, I64, I64, ctypes.c_int, P, ctypes.POINTER(P)]),
    "hm_ffn_info": (ctypes.c_int, [P, ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I32)]),
    "hm_ffn_destroy": (ctypes.c_int, [P]),
    "hm_ffn_workspace_bytes": (SZ, [P, I64]),
    "hm_ffn_forward": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I64, P, SZ, P]),
    "hm_ffn_forward_static": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I64, P]),
    "hm_ffn_block_workspace_bytes": (SZ, [P, I64]),
    "hm_ffn_block_forward": (ctypes.c_int, [P, P, I64, P, ctypes.c_float, I64, P, SZ, P]),
    "hm_ffn_gate_up": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I64, P, SZ, P]),
    "hm_ffn_down": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I64, P, SZ, P]),
    "hm_silu_mul": (ctypes.c_int, [P, I64, P, I64, I64, I64, I32, ctypes.c_int, P]),
    "hm_rmsnorm": (ctypes.c_int, [P, I64, P, I64, P, I64, I64, ctypes.c_float, ctypes.c_int, P]),
    "hm_residual_add2": (ctypes.c_int, [P, I64, P, I64, P, I64, I64, I64, ctypes.c_int, P]),
    "hm_residual_rmsnorm": (ctypes.c_int, [P, I64, P, I64, P, P, I64, I64, I64, ctypes.c_float, ctypes.c_int, P]),
    "hm_residual2_rmsnorm": (ctypes.c_int, [P, I64, P, I64, P, I64, P, P, I64, I64, I64, ctypes.c_float, ctypes.c_int, P]),
    "hm_residual_add2_mixed": (ctypes.c_int, [P, I64, P, I64, I32, P, I64, I32, I64, I64, ctypes.c_int, P]),
    "hm_find_nonfinite": (I64, [P, I64, I64, I64, ctypes.c_int, I32]),
    "hm_find_nonfinite_device": (ctypes.c_int, [P, I64, I64, I64, ctypes.c_int, I32, P, P]),
    "hm_partition_check": (ctypes.c_int, [I64, I64, I64]),
    "hm_partition_from_ratio": (ctypes.c_int, [I64, ctypes.c_double, I64, ctypes.POINTER(I64)]),
    "hm_split_type": (I32, [I32, I32, I32, I32, I32, I32]),
    "hm_layer_id": (I32, [ctypes.c_char_p]),
    "hm_split_table_create": (ctypes.c_int, [ctypes.POINTER(P)]),
    "hm_split_table_destroy": (ctypes.c_int, [P]),
    "hm_split_table_add_gemm": (ctypes.c_int, [P, I32, I32, I32, I32, I32, I32, I32, I32, I32, ctypes.POINTER(I32)]),
    "hm_split_table_add_gemv": (ctypes.c_int, [P, I32, I32, I32, I32, I32, I32, I32, I32]),
    "hm_split_table_find": (ctypes.c_int, [P, I32, I32, I32, I32, I32, P]),
    "hm_split_table_size": (I64, [P]),
    "hm_linear_split_workspace_bytes": (SZ, [P, P, P, I64, I64, I64]),
    "hm_linear_split": (ctypes.c_int, [P, P, P, P, I64, P, I64, I64, I64, I64, P, SZ, P]),
    "hm_merged_ffn_check": (ctypes.c_int, [I64, I64, I64, I64, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64)]),
    "hm_merged_ffn_supports": (I32, [I64, I64, I64, I64, I64, I64]),
}

_lib = None


def load():
    """Loads the in-tree library (once). Raises ImportError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python heteromega_amd/build.py` (or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return load().hm_last_error().decode("utf-8", "replace")


def check(status):
    if status != HM_OK:
        raise HMError(status, last_error())
