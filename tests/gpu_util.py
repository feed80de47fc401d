"""Helpers of the GPU parity tests: seeded inputs as exact 16-bit values, device transfer, and the
tolerance check against the float64 oracle."""

import ctypes

import numpy as np
import torch

# Parity bar for fp16 output: max|got-ref| / max|ref| <= 1e-2 and relative L2 <= 1e-3.
# bf16 output carries one bf16 rounding (~1.7e-3 rel-L2 by itself), so it uses the reference's own bar for a
# result with one bf16 rounding (kernels/gpu/tests/test_gpu_ffn.cpp:34): rel-L2 <= 5e-3.
TOL = {
    "fp16": {"max_rel": 1e-2, "rel_l2": 1e-3, "cos": 0.99999},
    "bf16": {"max_rel": 1e-2, "rel_l2": 5e-3, "cos": 0.99999},
}

TORCH = {"fp16": torch.float16, "bf16": torch.bfloat16}


def dev(a, device):
    # a fresh copy: a view such as a[None, :] has a zero stride that from_numpy would keep
    return torch.from_numpy(np.array(a, order="C", copy=True)).to(device)


def dev_bits(bits, dtype, device):
    return torch.from_numpy(np.array(bits, np.uint16, order="C", copy=True).view(np.int16)).view(TORCH[dtype]).to(device)


def host_f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def host_bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def make_x(oracle, rng, m, k, dtype, device, scale=1.0):
    """x ~ N(0, scale^2) rounded to dtype: (exact float64 values, device tensor)."""
    bits = oracle.to_bits((rng.standard_normal((m, k)) * scale).astype(np.float32), dtype)
    return oracle.from_bits(bits, dtype).astype(np.float64), dev_bits(bits, dtype, device)


def logical_to_device(w, dtype, device):
    q, s, z = w
    return dev(q, device), dev_bits(s, dtype, device), dev(z, device)


def assert_close(oracle, got, ref, dtype, tag=""):
    e = oracle.errors(got, ref)
    tol = TOL[dtype]
    print(f"{tag} {dtype}: max_rel={e['max_rel']:.2e} rel_l2={e['rel_l2']:.2e} cos={e['cos']:.7f} max_abs={e['max_abs']:.3e}", flush=True)
    assert np.all(np.isfinite(got)), tag
    assert e["max_rel"] <= tol["max_rel"] and e["rel_l2"] <= tol["rel_l2"] and e["cos"] >= tol["cos"], (tag, e)
    return e


def copy_device_bytes(ptr, nbytes):
    """Copies raw device memory (a plane of the repacked weights) to a host numpy array."""
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded (same SONAME)
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out = np.empty(nbytes, np.uint8)
    torch.cuda.synchronize()
    rc = hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), nbytes, 2)  # hipMemcpyDeviceToHost
    assert rc == 0, rc
    return out
