"""Builds oracle/_ref/libref_pack.so: the reference's own packing code (kernels/gpu/src/pack_w4a16.cpp, compiled
from where it lies under the reference tree, with its own header kernels/gpu/include/heteromega/gpu_ffn.hpp) and the
C interface oracle/ref_pack_c.cpp, against torch's C++ headers and libraries. Test infrastructure: the tests use it to
pin the packers byte for byte; nothing on the product path loads it. Does nothing when the reference tree is absent
(the GPU box); the built library travels with the tree.

Usage: python oracle/build_ref.py [reference root, default /root/reference]
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_ref")
OUT = os.path.join(OUT_DIR, "libref_pack.so")


def build(ref=None):
    ref = ref or os.environ.get("HM_REFERENCE_ROOT", "/root/reference")
    src = os.path.join(ref, "kernels", "gpu", "src", "pack_w4a16.cpp")
    inc = os.path.join(ref, "kernels", "gpu", "include")
    if not os.path.exists(src):
        print(f"build_ref: {src} is absent; oracle/_ref is not rebuilt", flush=True)
        return None
    import torch
    import torch.utils.cpp_extension as ext

    lib = ext.library_paths()[0]
    flags = ["-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-D__HIP_PLATFORM_AMD__",
             "-I/opt/rocm/include", f"-I{inc}", *[f"-I{p}" for p in ext.include_paths()]]
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ["g++", *flags, os.path.join(HERE, "ref_pack_c.cpp"), src, f"-L{lib}", "-lc10", "-ltorch", "-ltorch_cpu", f"-Wl,-rpath,{lib}",
           "-o", OUT + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build_ref failed:\n{res.stdout}\n{res.stderr}")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(sys.argv[1] if len(sys.argv) > 1 else None))
