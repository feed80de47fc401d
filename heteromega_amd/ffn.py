"""Host-side mirror of the reference's W4A16 FFN operator interface, over the C ABI (include/hm_w4a16.h).

Names and argument meanings follow kernels/gpu/include/heteromega/gpu_ffn.hpp (pack_w4a16, packed_tile_index,
packed_linear, gemv_w4a16, gemm_w4a16, silu_mul, residual_add2, GpuFfnModel) and npu/ffn/reference.py
(FFNPartition, ffn_partitioned). Errors surface as ValueError for bad arguments (the reference's
TORCH_CHECK / ValueError) and HMError for device failures. torch is used for device memory and streams only.
"""

import ctypes
import math
from numbers import Integral

import numpy as np
import torch

from . import _lib
from ._lib import HMError, check

kTileK = 128
kTileN = 64
kTileBytes = 4352

_DTYPES = {torch.bfloat16: _lib.HM_BF16, torch.float16: _lib.HM_FP16}
_TORCH_DTYPES = {_lib.HM_BF16: torch.bfloat16, _lib.HM_FP16: torch.float16}


def _hm_dtype(dtype):
    if isinstance(dtype, str):
        dtype = {"bf16": torch.bfloat16, "bfloat16": torch.bfloat16, "fp16": torch.float16, "float16": torch.float16}[dtype]
    if dtype not in _DTYPES:
        raise ValueError(f"activation dtype must be bfloat16 or float16, got {dtype}")
    return _DTYPES[dtype]


def _stream(stream, device=None):
    if stream is None:
        return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(int(stream))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _layout(layout):
    """GateUpLayout (gpu_ffn.hpp:43-46) by name."""
    try:
        return {"blocked": _lib.HM_GATE_UP_BLOCKED, "interleaved": _lib.HM_GATE_UP_INTERLEAVED}[layout]
    except KeyError:
        raise ValueError(f"gate_up layout must be 'blocked' or 'interleaved', got {layout!r}") from None


def _call(status):
    if status == _lib.HM_INVALID_ARGUMENT:
        raise ValueError(_lib.last_error())
    check(status)


def padded_rows(m):
    """Rows a reference GEMM input must hold (gpu_ffn.hpp:22-24). This engine needs no padding; kept for callers."""
    return (m + kTileK - 1) // kTileK * kTileK


# ---- reference 4352-byte tile format (host) -----------------------------------------------------

def packed_bytes(k, n):
    return _lib.load().hm_packed_bytes(k, n)


def packed_tile_index(c, r, tiles_k, tiles_n):
    """Position of tile (tile column c, tile row r) (pack_w4a16.cpp:100-107)."""
    idx = _lib.load().hm_packed_tile_index(c, r, tiles_k, tiles_n)
    if idx < 0:
        raise ValueError(f"packed_tile_index: tile ({c}, {r}) outside {tiles_k} x {tiles_n}")
    return idx


def _host_array(t, dtype):
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16 or t.dtype == torch.float16:
            t = t.view(torch.int16)
        t = t.numpy()
    return np.ascontiguousarray(np.asarray(t).astype(dtype, copy=False))


def pack_w4a16(qweight, scales, zeros):
    """Packs a [K, N] W4A16 matrix into the 4352-byte tile layout (pack_w4a16.cpp:9-66).
    qweight [K, N] uint8 0..15, scales [K/128, N] bf16 (torch bf16 tensor or uint16 bits), zeros [K/128, N]
    int8. Returns a flat uint8 numpy array."""
    q = _host_array(qweight, np.uint8)
    s = _host_array(scales, np.uint16)
    z = _host_array(zeros, np.int8)
    if q.ndim != 2:
        raise ValueError("pack_w4a16: qweight must be [K, N]")
    k, n = q.shape
    if s.shape != (k // kTileK, n) or z.shape != (k // kTileK, n):
        raise ValueError("pack_w4a16: scales and zeros must be [K/128, N]")
    nbytes = packed_bytes(k, n)
    if nbytes < 0:
        raise ValueError(f"pack_w4a16: K must be a multiple of 128 and N of 64, got {k}x{n}")
    out = np.empty(nbytes, np.uint8)
    _call(_lib.load().hm_pack_w4a16(q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p),
                                    z.ctypes.data_as(ctypes.c_void_p), k, n, out.ctypes.data_as(ctypes.c_void_p)))
    return out


def _awq(packed):
    p = _host_array(packed, np.int32)
    rows, cols8 = p.shape
    out = np.empty((rows, cols8 * 8), np.uint8)
    _call(_lib.load().hm_awq_unpack(p.ctypes.data_as(ctypes.c_void_p), rows, cols8, out.ctypes.data_as(ctypes.c_void_p)))
    return out


def awq_unpack_qweight(qweight):
    """AWQ qweight [In, Out/8] int32 -> [In, Out] uint8 (_unpack_awq_qweight, llama3_8b_w4a16_model.py:340-349)."""
    return _awq(qweight)


def awq_unpack_qzeros(qzeros):
    """AWQ qzeros [G, Out/8] int32 -> [G, Out] (_unpack_awq_qzeros, llama3_8b_w4a16_model.py:352-358)."""
    return _awq(qzeros)


def gptq_unpack_qweight(qweight):
    """GPTQ qweight [In/8, Out] int32 -> [In, Out] uint8: nibble i of word (r, o) is row 8r + i
    (_unpack_gptq_qweight then _unpack_packed_out_in2_to_in_out, llama3_8b_w4a16_model.py:361-378, :398-407)."""
    p = _host_array(qweight, np.int32)
    if p.ndim != 2:
        raise ValueError("gptq_unpack_qweight: qweight must be [In/8, Out]")
    rows8, cols = p.shape
    out = np.empty((rows8 * 8, cols), np.uint8)
    _call(_lib.load().hm_gptq_unpack(p.ctypes.data_as(ctypes.c_void_p), rows8, cols, out.ctypes.data_as(ctypes.c_void_p)))
    return out


def gptq_unpack_qzeros(qzeros, add_one=True):
    """GPTQ qzeros [G, Out/8] int32 -> [G, Out] uint8, plus one when add_one (1..16; _unpack_gptq_qzeros,
    llama3_8b_w4a16_model.py:381-395, which returns the transpose [Out, G])."""
    p = _host_array(qzeros, np.int32)
    if p.ndim != 2:
        raise ValueError("gptq_unpack_qzeros: qzeros must be [G, Out/8]")
    groups, cols8 = p.shape
    out = np.empty((groups, cols8 * 8), np.uint8)
    _call(_lib.load().hm_gptq_unpack_zeros(p.ctypes.data_as(ctypes.c_void_p), groups, cols8, 1 if add_one else 0,
                                           out.ctypes.data_as(ctypes.c_void_p)))
    return out


# ---- repacked matrices ------------------------------------------------------------------------------

class RepackedMatrix:
    """One [K, N] W4A16 matrix in the device strip layout (hm_weights)."""

    def __init__(self, handle, device):
        self._h = handle
        self.device = device
        K, N, G, D, B = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int64()
        check(_lib.load().hm_weights_info(handle, ctypes.byref(K), ctypes.byref(N), ctypes.byref(G), ctypes.byref(D), ctypes.byref(B)))
        self.k, self.n, self.group, self.dtype, self.device_bytes = K.value, N.value, G.value, _TORCH_DTYPES[D.value], B.value
        self.fused = False  # a fused gate_up matrix (from_gate_up_tiles): n = 2 x channels

    @classmethod
    def from_tiles(cls, tiles, packed_k, packed_n, k=None, n=None, dtype=torch.bfloat16, stream=None):
        """The leading [k, n] block of a reference-packed [packed_k, packed_n] matrix held in device memory."""
        k = packed_k if k is None else k
        n = packed_n if n is None else n
        if not tiles.is_cuda or tiles.dtype != torch.uint8 or not tiles.is_contiguous() or tiles.numel() != packed_bytes(packed_k, packed_n):
            raise ValueError(f"from_tiles: expected contiguous device uint8 of {packed_bytes(packed_k, packed_n)} bytes")
        h = ctypes.c_void_p()
        _call(_lib.load().hm_weights_from_tiles(_ptr(tiles), packed_k, packed_n, k, n, _hm_dtype(dtype), _stream(stream, tiles.device),
                                                ctypes.byref(h)))
        return cls(h, tiles.device)

    @classmethod
    def from_logical(cls, q, scales, zeros, group, dtype=torch.bfloat16, stream=None):
        """From device tensors q [K, N] uint8, scales [K/group, N] (dtype), zeros [K/group, N] uint8."""
        for t in (q, scales, zeros):
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError("from_logical: tensors must be contiguous device tensors")
        if scales.dtype != dtype and scales.dtype not in (torch.int16, torch.uint16):
            raise ValueError("from_logical: scales must have the activation dtype")
        k, n = q.shape
        h = ctypes.c_void_p()
        _call(_lib.load().hm_weights_from_logical(_ptr(q), _ptr(scales), _ptr(zeros), k, n, group, _hm_dtype(dtype),
                                                  _stream(stream, q.device), ctypes.byref(h)))
        return cls(h, q.device)

    @classmethod
    def from_gate_up_tiles(cls, gate_up, packed_k, stored, k=None, channels=None, layout="interleaved", dtype=torch.bfloat16, stream=None):
        """The reference's fused gate_up tensor, packed [packed_k, 2 * stored] in `layout` order ("interleaved": per 64
        channels their gate columns then their up columns; "blocked": gate | up), as FfnSliceWeights.gate_up holds it
        (gpu_ffn.hpp:43-71). The result serves packed_linear_swiglu over channels [0, channels)."""
        k = packed_k if k is None else k
        channels = stored if channels is None else channels
        if not gate_up.is_cuda or gate_up.dtype != torch.uint8 or not gate_up.is_contiguous() or gate_up.numel() != packed_bytes(packed_k, 2 * stored):
            raise ValueError(f"from_gate_up_tiles: expected contiguous device uint8 of {packed_bytes(packed_k, 2 * stored)} bytes")
        h = ctypes.c_void_p()
        _call(_lib.load().hm_weights_from_gate_up_tiles(_ptr(gate_up), packed_k, stored, k, channels, _layout(layout), _hm_dtype(dtype),
                                                        _stream(stream, gate_up.device), ctypes.byref(h)))
        m = cls(h, gate_up.device)
        m.fused = True
        return m

    def dequantize(self, transposed=True, stream=None):
        """round((q - z) * s) in the activation type: [N, K] (QuantizedLinearImpl::dequantize_packed's orientation,
        unified_llm_w4a16.cpp:710-790) or [K, N]."""
        shape = (self.n, self.k) if transposed else (self.k, self.n)
        out = torch.empty(shape, dtype=self.dtype, device=self.device)
        _call(_lib.load().hm_weights_dequantize(self._h, _ptr(out), out.stride(0), 1 if transposed else 0, _stream(stream, self.device)))
        return out

    @classmethod
    def concat(cls, parts, stream=None):
        """The columns of matrices with the same K, group and dtype side by side, [K, sum of N]: an attention
        block's Q, K and V projections as one launch (the reference reuses only the prepared input,
        GemmInputReuse, gpu_ffn.hpp:117-127). The parts stay valid and owned by the caller."""
        if not parts:
            raise ValueError("concat: no parts")
        arr = (ctypes.c_void_p * len(parts))(*[p._h for p in parts])
        h = ctypes.c_void_p()
        _call(_lib.load().hm_weights_concat(arr, len(parts), _stream(stream, parts[0].device), ctypes.byref(h)))
        return cls(h, parts[0].device)

    def to_logical(self, stream=None):
        q = torch.empty((self.k, self.n), dtype=torch.uint8, device=self.device)
        s = torch.empty((self.k // self.group, self.n), dtype=self.dtype, device=self.device)
        z = torch.empty((self.k // self.group, self.n), dtype=torch.uint8, device=self.device)
        _call(_lib.load().hm_weights_to_logical(self._h, _ptr(q), _ptr(s), _ptr(z), _stream(stream, self.device)))
        return q, s, z

    def planes(self):
        """(quant_ptr, quant_bytes, meta_ptr, meta_bytes) of the device planes."""
        qp, qb, mp, mb = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_void_p(), ctypes.c_int64()
        check(_lib.load().hm_weights_planes(self._h, ctypes.byref(qp), ctypes.byref(qb), ctypes.byref(mp), ctypes.byref(mb)))
        return qp.value, qb.value, mp.value, mb.value

    def workspace_bytes(self, m, k=None, n=None):
        return _lib.load().hm_linear_workspace_bytes(self._h, m, self.k if k is None else k, self.n if n is None else n)

    def close(self):
        if self._h:
            _lib.load().hm_weights_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    return torch.empty(nbytes + 256, dtype=torch.uint8, device=device)


def _aligned(ws, nbytes):
    if ws is None:
        return ctypes.c_void_p(0), 0
    base = ws.data_ptr()
    off = (-base) % 256
    return ctypes.c_void_p(base + off), ws.numel() - off


def packed_linear(out, inp, w, k=None, n=None, col_begin=0, stream=None, workspace=None):
    """out[M, n] = inp[M, k] @ W[:k, col_begin:col_begin + n] (heteromega::packed_linear, gpu_ffn.hpp:196-199,
    with the reference GEMV's start_col). M <= 16 runs the decode GEMV, larger M the MFMA GEMM."""
    k = w.k if k is None else k
    n = w.n if n is None else n
    if inp.dim() != 2 or inp.size(1) < k or inp.stride(1) != 1:
        raise ValueError(f"packed_linear: input must be [M, >= {k}] with unit column stride")
    m = inp.size(0)
    if out.dim() != 2 or out.size(0) != m or out.size(1) < n or out.stride(1) != 1:
        raise ValueError(f"packed_linear: output must be [M, >= {n}]")
    if inp.dtype != w.dtype or out.dtype != w.dtype:
        raise ValueError(f"packed_linear: input and output must be {w.dtype}")
    need = w.workspace_bytes(m, k, n)
    if workspace is None:
        workspace = _workspace(need, inp.device)
    wp, wb = _aligned(workspace, need)
    _call(_lib.load().hm_linear(w._h, _ptr(out), out.stride(0), _ptr(inp), inp.stride(0), m, k, n, col_begin, wp, wb,
                                _stream(stream, inp.device)))
    return out


def packed_linear_k_split(out, inp, w0, w1, k0=None, k1=None, n=None, stream=None, workspace=None):
    """K split over a pair of packed matrices (hetero_matmul_out_gemm_packed_K / hetero_matmul_out_gemv_packed_K,
    hetero_compute.cpp:282-447, 633-805, GPU-only): out = round(round(inp[:, :k0] @ W0) + round(inp[:, k0:k0 + k1] @ W1)),
    the reference's sum of the two shares' outputs. Both shares run on the GPU; the second adds into out."""
    k0 = w0.k if k0 is None else k0
    k1 = w1.k if k1 is None else k1
    n = min(w0.n, w1.n) if n is None else n
    if inp.dim() != 2 or inp.size(1) < k0 + k1 or inp.stride(1) != 1:
        raise ValueError(f"packed_linear_k_split: input must be [M, >= {k0 + k1}] with unit column stride")
    m = inp.size(0)
    if out.dim() != 2 or out.size(0) != m or out.size(1) < n or out.stride(1) != 1:
        raise ValueError(f"packed_linear_k_split: output must be [M, >= {n}]")
    if w0.dtype != w1.dtype or inp.dtype != w0.dtype or out.dtype != w0.dtype:
        raise ValueError(f"packed_linear_k_split: input, output and both shares must be {w0.dtype}")
    lib = _lib.load()
    need = lib.hm_linear_k_split_workspace_bytes(w0._h, w1._h, m, k0, k1, n)
    if workspace is None:
        workspace = _workspace(need, inp.device)
    wp, wb = _aligned(workspace, need)
    _call(lib.hm_linear_k_split(w0._h, w1._h, _ptr(out), out.stride(0), _ptr(inp), inp.stride(0), m, k0, k1, n, wp, wb,
                                _stream(stream, inp.device)))
    return out


def packed_linear_swiglu(act, inp, w, k=None, channels=None, stream=None, workspace=None):
    """act[M, e - b] = SiLU(inp @ Wg[:k, b:e]) * (inp @ Wu[:k, b:e]) on a fused gate_up matrix (from_gate_up_tiles):
    hipkernels::w4a16_gemm_fused_packed_tiles with fuse_activation (w4a16_gemm_packed.cu:549-578), any M.
    channels=(b, e), all by default."""
    if not w.fused:
        raise ValueError("packed_linear_swiglu: needs a fused gate_up matrix (RepackedMatrix.from_gate_up_tiles)")
    k = w.k if k is None else k
    b, e = (0, w.n // 2) if channels is None else channels
    if inp.dim() != 2 or inp.size(1) < k or inp.stride(1) != 1:
        raise ValueError(f"packed_linear_swiglu: input must be [M, >= {k}] with unit column stride")
    m = inp.size(0)
    if act.dim() != 2 or act.size(0) != m or act.size(1) < e - b or act.stride(1) != 1:
        raise ValueError(f"packed_linear_swiglu: output must be [M, >= {e - b}]")
    lib = _lib.load()
    need = lib.hm_linear_swiglu_workspace_bytes(w._h, m, k, e - b)
    if workspace is None:
        workspace = _workspace(need, inp.device)
    wp, wb = _aligned(workspace, need)
    _call(lib.hm_linear_swiglu(w._h, _ptr(act), act.stride(0), _ptr(inp), inp.stride(0), m, k, b, e, wp, wb, _stream(stream, inp.device)))
    return act


def gemv_w4a16(out, x, w, k=None, n=None, col_begin=0, stream=None):
    """M = 1 (heteromega::gemv_w4a16, gpu_ffn.hpp:99-103)."""
    if x.dim() != 2 or x.size(0) != 1:
        raise ValueError("gemv_w4a16: x must be [1, K]")
    return packed_linear(out, x, w, k, n, col_begin, stream)


def gemm_w4a16(out, x, w, k=None, n=None, stream=None):
    """M > 1 (heteromega::gemm_w4a16, gpu_ffn.hpp:105-110)."""
    return packed_linear(out, x, w, k, n, 0, stream)


# ---- elementwise ------------------------------------------------------------------------------------

def silu_mul(gate_up, act, layout="blocked", stream=None):
    """act = SiLU(gate) * up, fp32 math, one rounding (heteromega::silu_mul, silu_mul.cu:34-57)."""
    lay = {"blocked": _lib.HM_GATE_UP_BLOCKED, "interleaved": _lib.HM_GATE_UP_INTERLEAVED}[layout]
    if gate_up.dim() != 2 or act.dim() != 2 or gate_up.size(0) != act.size(0) or gate_up.size(1) != 2 * act.size(1):
        raise ValueError("silu_mul: gate_up must be [M, 2n] and act [M, n]")
    if gate_up.dtype != act.dtype:
        raise ValueError("silu_mul: dtypes differ")
    _call(_lib.load().hm_silu_mul(_ptr(gate_up), gate_up.stride(0), _ptr(act), act.stride(0), act.size(0), act.size(1), lay,
                                  _hm_dtype(act.dtype), _stream(stream, act.device)))
    return act


def rmsnorm(out, x, weight, eps=1e-5, stream=None):
    """out = x * rsqrt(mean(x^2) + eps) * weight (launch_rmsnorm, rmsnorm.cu:65-103)."""
    _call(_lib.load().hm_rmsnorm(_ptr(out), out.stride(0), _ptr(x), x.stride(0), _ptr(weight), x.size(0), x.size(1), eps,
                                 _hm_dtype(x.dtype), _stream(stream, x.device)))
    return out


def residual_add2(x, y_g, y_n=None, stream=None):
    """x += y_g + y_n (heteromega::residual_add2, residual_add.cu:9-73); y_n may be None. Each partial is of x's
    type or float32 (then both must be given, as in the reference)."""
    if (y_g is not None and y_g.dtype == torch.float32) or (y_n is not None and y_n.dtype == torch.float32):
        if y_g is None or y_n is None:
            raise ValueError("residual_add2: fp32 partials need both y_g and y_n")
        _call(_lib.load().hm_residual_add2_mixed(_ptr(x), x.stride(0), _ptr(y_g), y_g.stride(0), int(y_g.dtype == torch.float32), _ptr(y_n),
                                                 y_n.stride(0), int(y_n.dtype == torch.float32), x.size(0), x.size(1), _hm_dtype(x.dtype),
                                                 _stream(stream, x.device)))
        return x
    _call(_lib.load().hm_residual_add2(_ptr(x), x.stride(0), _ptr(y_g), y_g.stride(0) if y_g is not None else 0, _ptr(y_n),
                                       y_n.stride(0) if y_n is not None else 0, x.size(0), x.size(1), _hm_dtype(x.dtype),
                                       _stream(stream, x.device)))
    return x


def residual_rmsnorm(x, y, weight, normed, eps=1e-5, stream=None):
    """x += y, then normed = RMSNorm(x) * weight, in one dispatch (residual_norm.cu:25-98 without GEMM prep)."""
    _call(_lib.load().hm_residual_rmsnorm(_ptr(x), x.stride(0), _ptr(y), y.stride(0), _ptr(weight), _ptr(normed), normed.stride(0),
                                          x.size(0), x.size(1), eps, _hm_dtype(x.dtype), _stream(stream, x.device)))
    return normed


def residual_norm(x, a, b, weight, normed, eps=1e-5, stream=None):
    """x = round((x + a) + b), then normed = RMSNorm(x) * weight, in one dispatch (heteromega::residual_norm_bf16,
    residual_norm.cu:25-106, without its GEMM input prep). a and b may be None; without a, x is left as it is."""
    _call(_lib.load().hm_residual2_rmsnorm(_ptr(x), x.stride(0), _ptr(a), a.stride(0) if a is not None else 0, _ptr(b),
                                           b.stride(0) if b is not None else 0, _ptr(weight), _ptr(normed), normed.stride(0), x.size(0),
                                           x.size(1), eps, _hm_dtype(x.dtype), _stream(stream, x.device)))
    return normed


kFiniteSampleStride = 64


def find_nonfinite(t, sampled=False, stream=None):
    """Index of the first checked inf/NaN element of a [rows, columns] fp16/bf16 tensor, or -1: every element, or
    every row at one in kFiniteSampleStride columns (heteromega::find_nonfinite_bf16 with FiniteCheck::kFull /
    kSampled, merged_ffn_contract.hpp:13-39). A device tensor is scanned on the GPU where it lies (one int64
    comes back); a host tensor on the host."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("find_nonfinite: a [rows, columns] tensor with a contiguous last dimension")
    L = _lib.load()
    if t.is_cuda:
        first = torch.empty((1,), dtype=torch.int64, device=t.device)
        _call(L.hm_find_nonfinite_device(_ptr(t), t.size(0), t.size(1), t.stride(0), _hm_dtype(t.dtype), int(bool(sampled)), _ptr(first),
                                         _stream(stream, t.device)))
        return int(first.item())
    return int(L.hm_find_nonfinite(_ptr(t), t.size(0), t.size(1), t.stride(0), _hm_dtype(t.dtype), int(bool(sampled))))


# ---- FFN layer --------------------------------------------------------------------------------------

class FfnLayer:
    """One SwiGLU FFN layer in the strip layout (hm_ffn): gate and up fused per 16 channels, down as is."""

    def __init__(self, handle, device):
        self._h = handle
        self.device = device
        H, I, G, D = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        check(_lib.load().hm_ffn_info(handle, ctypes.byref(H), ctypes.byref(I), ctypes.byref(G), ctypes.byref(D)))
        self.hidden, self.inter, self.group, self.dtype = H.value, I.value, G.value, _TORCH_DTYPES[D.value]
        self._ws = {}

    @classmethod
    def from_tiles(cls, gate, up, down, hidden, inter, dtype=torch.bfloat16, stream=None, packed_hidden=None, packed_inter=None):
        """From reference-packed device matrices gate [H, I], up [H, I], down [I, H] (GpuFfnModel::add_layer).
        packed_hidden / packed_inter: the packed extents when the matrices were padded (padPackedWeights,
        llama3_8b_w4a16_model.py:546-608); the layer is their leading [hidden, inter] block."""
        ph = hidden if packed_hidden is None else packed_hidden
        pi = inter if packed_inter is None else packed_inter
        for t, (k, n) in ((gate, (ph, pi)), (up, (ph, pi)), (down, (pi, ph))):
            if not t.is_cuda or t.dtype != torch.uint8 or not t.is_contiguous():
                raise ValueError("from_tiles: packed matrices must be contiguous device uint8 tensors")
            if packed_bytes(k, n) < 0 or t.numel() != packed_bytes(k, n):
                raise ValueError(f"from_tiles: a packed [{k}, {n}] matrix has {packed_bytes(k, n)} bytes, got {t.numel()}")
        h = ctypes.c_void_p()
        _call(_lib.load().hm_ffn_from_tiles_padded(_ptr(gate), _ptr(up), _ptr(down), hidden, inter, ph, pi, _hm_dtype(dtype),
                                                   _stream(stream, gate.device), ctypes.byref(h)))
        return cls(h, gate.device)

    @classmethod
    def from_gate_up_tiles(cls, gate_up, down, hidden, inter, stored=None, layout="interleaved", dtype=torch.bfloat16, stream=None):
        """From the reference's fused-FFN tensors (FfnSliceWeights, gpu_ffn.hpp:55-71; gemm_w4a16_ffn's inputs):
        gate_up packed [hidden, 2 * stored] in `layout` order and down packed [stored, hidden]; the layer is channels
        [0, inter) of them (prefix)."""
        stored = inter if stored is None else stored
        for t, (k, n) in ((gate_up, (hidden, 2 * stored)), (down, (stored, hidden))):
            if not t.is_cuda or t.dtype != torch.uint8 or not t.is_contiguous():
                raise ValueError("from_gate_up_tiles: packed matrices must be contiguous device uint8 tensors")
            if packed_bytes(k, n) < 0 or t.numel() != packed_bytes(k, n):
                raise ValueError(f"from_gate_up_tiles: a packed [{k}, {n}] matrix has {packed_bytes(k, n)} bytes, got {t.numel()}")
        h = ctypes.c_void_p()
        _call(_lib.load().hm_ffn_from_gate_up_tiles(_ptr(gate_up), _ptr(down), hidden, inter, stored, _layout(layout), _hm_dtype(dtype),
                                                    _stream(stream, gate_up.device), ctypes.byref(h)))
        return cls(h, gate_up.device)

    @classmethod
    def from_logical(cls, gate, up, down, group, dtype=torch.bfloat16, stream=None):
        """gate, up: (q [H, I] uint8, s [H/g, I] dtype, z [H/g, I] uint8); down: (q [I, H], s [I/g, H], z [I/g, H])."""
        hidden, inter = gate[0].shape
        args = []
        for q, s, z in (gate, up, down):
            for t in (q, s, z):
                if not t.is_cuda or not t.is_contiguous():
                    raise ValueError("from_logical: tensors must be contiguous device tensors")
            args += [_ptr(q), _ptr(s), _ptr(z)]
        h = ctypes.c_void_p()
        _call(_lib.load().hm_ffn_from_logical(*args, hidden, inter, group, _hm_dtype(dtype), _stream(stream, gate[0].device),
                                              ctypes.byref(h)))
        return cls(h, gate[0].device)

    def workspace_bytes(self, max_m):
        return _lib.load().hm_ffn_workspace_bytes(self._h, max_m)

    def workspace(self, max_m, stream=None):
        """Per-stream workspace, grown as needed (the reference keeps GpuFfnBuffers per stream, gpu_ffn.cpp:142-156)."""
        key = _stream(stream, self.device).value
        need = self.workspace_bytes(max_m)
        ws = self._ws.get(key)
        if ws is None or ws.numel() < need + 256:
            ws = torch.empty(need + 256, dtype=torch.uint8, device=self.device)
            self._ws[key] = ws
        return ws

    def _channels(self, channels):
        return (0, self.inter) if channels is None else channels

    def forward(self, x, y=None, channels=None, stream=None, workspace=None):
        """y [M, H] = FFN of x [M, H] over channels [b, e) (all by default)."""
        b, e = self._channels(channels)
        m = x.size(0)
        if y is None:
            y = torch.empty((m, self.hidden), dtype=x.dtype, device=x.device)
        if workspace is None:
            workspace = self.workspace(m, stream)
        wp, wb = _aligned(workspace, self.workspace_bytes(m))
        _call(_lib.load().hm_ffn_forward(self._h, _ptr(y), y.stride(0), _ptr(x), x.stride(0), m, b, e, wp, wb, _stream(stream, x.device)))
        return y

    def block_workspace_bytes(self, max_m):
        return _lib.load().hm_ffn_block_workspace_bytes(self._h, max_m)

    def block_forward(self, x, norm_weight, eps=1e-5, stream=None, workspace=None):
        """In place: x [M, H] += FFN(RMSNorm(x) * norm_weight), the pre-norm FFN block of a layer stack
        (unified_llm_w4a16.cpp:2867-2892 with the layer-boundary norm and residual of residual_norm.cu:25-98).

        Equal bit for bit to rmsnorm, forward and residual_add2 in sequence; one row runs as two launches."""
        if norm_weight.numel() != self.hidden or norm_weight.dtype != x.dtype or not norm_weight.is_contiguous():
            raise ValueError(f"norm_weight must be a contiguous {x.dtype} vector of {self.hidden} elements")
        m = x.size(0)
        need = self.block_workspace_bytes(m)
        if workspace is None:
            key = ("block", _stream(stream, self.device).value)
            workspace = self._ws.get(key)
            if workspace is None or workspace.numel() < need + 256:
                workspace = torch.empty(need + 256, dtype=torch.uint8, device=self.device)
                self._ws[key] = workspace
        wp, wb = _aligned(workspace, need)
        _call(_lib.load().hm_ffn_block_forward(self._h, _ptr(x), x.stride(0), _ptr(norm_weight), eps, m, wp, wb,
                                               _stream(stream, x.device)))
        return x

    def gate_up(self, x, act=None, channels=None, stream=None):
        b, e = self._channels(channels)
        m = x.size(0)
        if act is None:
            act = torch.empty((m, e - b), dtype=x.dtype, device=x.device)
        ws = self.workspace(m, stream)
        wp, wb = _aligned(ws, self.workspace_bytes(m))
        _call(_lib.load().hm_ffn_gate_up(self._h, _ptr(act), act.stride(0), _ptr(x), x.stride(0), m, b, e, wp, wb,
                                         _stream(stream, x.device)))
        return act

    def down(self, act, y=None, channels=None, stream=None):
        b, e = self._channels(channels)
        m = act.size(0)
        if y is None:
            y = torch.empty((m, self.hidden), dtype=act.dtype, device=act.device)
        ws = self.workspace(m, stream)
        wp, wb = _aligned(ws, self.workspace_bytes(m))
        _call(_lib.load().hm_ffn_down(self._h, _ptr(y), y.stride(0), _ptr(act), act.stride(0), m, b, e, wp, wb, _stream(stream, act.device)))
        return y

    def close(self):
        if self._h:
            _lib.load().hm_ffn_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- partition descriptor ---------------------------------------------------------------------------

class FFNPartition:
    """The other device owns channels [0, npu_channels), the GPU owns the rest (reference.py:121-151).
    On this build both shares run on the GPU; npu_channels = 0 is the GPU-only layer."""

    def __init__(self, intermediate_channels, npu_channels, alignment=128):
        for name, v in (("intermediate_channels", intermediate_channels), ("alignment", alignment)):
            if isinstance(v, bool) or not isinstance(v, Integral) or v <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if isinstance(npu_channels, bool) or not isinstance(npu_channels, Integral):
            raise ValueError("npu_channels must be an integer")
        _call(_lib.load().hm_partition_check(intermediate_channels, npu_channels, alignment))
        self.intermediate_channels = int(intermediate_channels)
        self.npu_channels = int(npu_channels)
        self.alignment = int(alignment)

    @classmethod
    def from_ratio(cls, intermediate_channels, npu_ratio, alignment=128):
        if isinstance(intermediate_channels, bool) or not isinstance(intermediate_channels, Integral) or intermediate_channels <= 0:
            raise ValueError("intermediate_channels must be a positive integer")
        if not math.isfinite(npu_ratio):
            raise ValueError("npu_ratio must be finite and in [0, 1]")
        out = ctypes.c_int64()
        _call(_lib.load().hm_partition_from_ratio(intermediate_channels, float(npu_ratio), alignment, ctypes.byref(out)))
        return cls(intermediate_channels, out.value, alignment)

    @property
    def slices(self):
        return {"npu": (0, self.npu_channels), "gpu": (self.npu_channels, self.intermediate_channels)}


def ffn_partitioned(layer, x, partition, stream=None):
    """(reduced, partials): each share of the channel split run on the GPU one after the other, then summed with
    one rounding (reference.py:200-221; merged_ffn.cpp:301-432 with the NPU leg on the GPU). Empty shares give
    zero partials."""
    if partition.intermediate_channels != layer.inter:
        raise ValueError("partition width must equal the intermediate FFN width")
    partials = {}
    for dev, (b, e) in partition.slices.items():
        if b == e:
            partials[dev] = torch.zeros((x.size(0), layer.hidden), dtype=x.dtype, device=x.device)
        else:
            partials[dev] = layer.forward(x, channels=(b, e), stream=stream)
    reduced = torch.zeros((x.size(0), layer.hidden), dtype=x.dtype, device=x.device)
    residual_add2(reduced, partials["gpu"], partials["npu"], stream=stream)
    return reduced, partials


def ffn_row_split(layer, x, y, other_rows, stream=None):
    """Row (M) split of hetero_compute.cpp:189-259: the GPU takes rows [0, M - other_rows), the other device
    the tail; here both run on the GPU. Rows are independent: the result has the unsplit FFN's bits when no
    part's GEMM splits its K range (small grids split: under 128 workgroups, 4-wave grids under 512, and long-K
    down projections whose 128 x 256 grid is under 128 workgroups; e.g. a Llama-3-8B part of 1152 rows or more,
    or a Qwen2.5-14B part of 1024 or more, does not), and equals it within rounding otherwise."""
    m = x.size(0)
    if not 0 <= other_rows <= m:
        raise ValueError("row split outside [0, M]")
    g = m - other_rows
    if g > 0:
        layer.forward(x[:g], y[:g], stream=stream)
    if other_rows > 0:
        layer.forward(x[g:], y[g:], stream=stream)
    return y


# ---- model integration ------------------------------------------------------------------------------

class GpuFfnModel:
    """The GPU FFN of every layer of a model (GpuFfnModel, gpu_ffn.hpp:219-242). A forward pass uses the first
    s_prefill channels when M > 1 and the first s_decode channels when M == 1; the rest is the other device's
    share, which this class does not compute."""

    def __init__(self, dtype=torch.bfloat16):
        self.dtype = dtype
        self._layers = []
        self.s_prefill = 0
        self.s_decode = 0

    def add_layer(self, gate, up, down, hidden, inter, stream=None):
        """From reference-packed device matrices gate [H, I], up [H, I] and down [I, H]."""
        if self._layers and (self._layers[0].hidden != hidden or self._layers[0].inter != inter):
            raise ValueError("GpuFfnModel.add_layer: all layers must have the same shape")
        self._layers.append(FfnLayer.from_tiles(gate, up, down, hidden, inter, self.dtype, stream))
        if self.s_prefill == 0:
            self.s_prefill = self.s_decode = inter

    def add_layer_logical(self, gate, up, down, group, stream=None):
        self.append(FfnLayer.from_logical(gate, up, down, group, self.dtype, stream))

    def append(self, layer):
        """Adds a built FfnLayer (of this model's dtype and shape)."""
        if layer.dtype != self.dtype:
            raise ValueError(f"GpuFfnModel.append: layer dtype {layer.dtype} differs from the model's {self.dtype}")
        if self._layers and (self._layers[0].hidden != layer.hidden or self._layers[0].inter != layer.inter):
            raise ValueError("GpuFfnModel.add_layer: all layers must have the same shape")
        self._layers.append(layer)
        if self.s_prefill == 0:
            self.s_prefill = self.s_decode = layer.inter

    def set_split(self, s_prefill, s_decode):
        if not self._layers:
            raise ValueError("GpuFfnModel.set_split: add the layers first")
        inter = self._layers[0].inter
        for s in (s_prefill, s_decode):
            if not (0 < s <= inter and s % kTileK == 0):
                raise ValueError(f"GpuFfnModel.set_split: channels must be a multiple of 128 in (0, {inter}], got {s}")
        self.s_prefill, self.s_decode = s_prefill, s_decode

    def layers(self):
        return len(self._layers)

    def layer(self, i):
        return self._layers[i]

    def channels(self, m):
        return self.s_prefill if m > 1 else self.s_decode

    def forward(self, layer, x_norm, y, stream=None):
        if not 0 <= layer < len(self._layers):
            raise ValueError(f"GpuFfnModel.forward: no layer {layer}")
        return self._layers[layer].forward(x_norm, y, channels=(0, self.channels(x_norm.size(0))), stream=stream)


__all__ = [
    "HMError", "kTileK", "kTileN", "kTileBytes", "padded_rows", "packed_bytes", "packed_tile_index", "pack_w4a16",
    "awq_unpack_qweight", "awq_unpack_qzeros", "gptq_unpack_qweight", "gptq_unpack_qzeros", "RepackedMatrix", "packed_linear", "packed_linear_k_split",
    "packed_linear_swiglu", "gemv_w4a16", "gemm_w4a16", "silu_mul",
    "rmsnorm", "residual_add2", "residual_rmsnorm", "residual_norm", "kFiniteSampleStride", "find_nonfinite", "FfnLayer", "FFNPartition", "ffn_partitioned", "ffn_row_split", "GpuFfnModel",
]
