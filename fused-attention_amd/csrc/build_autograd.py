"""Builds the C++ autograd op (fa_autograd.cpp) into fused-attention_amd/fa_autograd<EXT_SUFFIX>.

    python3 fused-attention_amd/csrc/build_autograd.py

A torch extension compiled with g++ against the installed torch (its headers, its C++ ABI flag,
its c10/c10_hip/torch libraries) and linked to libfa.so in the same folder (run-time path
$ORIGIN), so build libfa.so first (make -C fused-attention_amd/csrc).  No device code: it only
calls the C ABI of include/fa.h.
"""

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
INCLUDE = os.path.join(os.path.dirname(PKG), "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def main():
    import torch
    tdir = os.path.dirname(torch.__file__)
    out = os.path.join(PKG, "fa_autograd" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(os.path.join(PKG, "libfa.so")):
        sys.exit("build libfa.so first: make -C fused-attention_amd/csrc")
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=fa_autograd",
           f"-I{INCLUDE}", f"-I{ROCM}/include", f"-I{tdir}/include",
           f"-I{tdir}/include/torch/csrc/api/include", f"-I{sysconfig.get_paths()['include']}",
           os.path.join(HERE, "fa_autograd.cpp"), "-o", out + ".tmp",
           f"-L{tdir}/lib", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_python",
           f"-L{PKG}", "-lfa", "-Wl,-rpath,$ORIGIN"]
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(out + ".tmp", out)
    print(f"wrote {out}", flush=True)


if __name__ == "__main__":
    main()
