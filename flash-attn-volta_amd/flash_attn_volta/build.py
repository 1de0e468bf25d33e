"""In-tree build of the gfx950 C-ABI library ``libfa_mi355x.so`` and of
the C++ autograd node ``_fa_torch`` (a client of that library).

    python -m flash_attn_volta.build         (from flash-attn-volta_amd/)

hipcc cross-compiles for gfx950 on a machine without a GPU.  Every HIP
source is compiled with packed-fp32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops).  ``_fa_torch`` is host
C++ against the installed torch's headers and libraries (g++), linked to
``libfa_mi355x.so`` beside it.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                  # flash-attn-volta_amd/
CSRC = os.path.join(ROOT, "csrc")
SOURCES = [os.path.join(CSRC, "fa_api.hip")]
# The C-ABI header (fa_mi355x.h): the repository's include/ directory, or the
# directory named by FA_MI355X_INCLUDE when the package is built elsewhere.
INCLUDE_DIR = os.environ.get("FA_MI355X_INCLUDE",
                             os.path.join(os.path.dirname(ROOT), "include"))
HEADERS = [os.path.join(CSRC, f) for f in ("fa_common.hpp", "fa_fwd.hpp", "fa_bwd.hpp", "fa_rope.hpp")]
OUT = os.path.join(PKG_DIR, "libfa_mi355x.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in VGPRs (no AGPR<->VGPR copies around softmax)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    p = os.path.join(rocm, "bin", "hipcc")
    return p if os.path.exists(p) else "hipcc"


def build_library(verbose: bool = True) -> str:
    """Compile libfa_mi355x.so in place (always recompiles) and return its path."""
    tmp = OUT + ".tmp"
    header = os.path.join(INCLUDE_DIR, "fa_mi355x.h")
    if not os.path.exists(header):
        raise RuntimeError(f"{header} not found: set FA_MI355X_INCLUDE to the directory "
                           "holding the C-ABI header")
    cmd = [hipcc()] + HIPCC_FLAGS + ["-I", INCLUDE_DIR] + SOURCES + ["-o", tmp]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


TORCH_EXT_SRC = os.path.join(CSRC, "fa_torch.cpp")
TORCH_EXT_OUT = os.path.join(PKG_DIR, "_fa_torch.so")


def build_torch_ext(verbose: bool = True) -> str:
    """Compile the C++ autograd node _fa_torch.so in place (always
    recompiles; needs libfa_mi355x.so built first) and return its path."""
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths, library_paths
    if not os.path.exists(OUT):
        raise RuntimeError(f"{OUT} is not built: build_library() first")
    tmp = TORCH_EXT_OUT + ".tmp"
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_fa_torch"]
    for d in include_paths() + [os.path.join(rocm, "include"), sysconfig.get_paths()["include"],
                                INCLUDE_DIR]:
        cmd += ["-I", d]
    cmd += [TORCH_EXT_SRC]
    for d in library_paths():
        cmd += ["-L", d]
    cmd += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
            "-L", PKG_DIR, "-lfa_mi355x", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, TORCH_EXT_OUT)
    return TORCH_EXT_OUT


if __name__ == "__main__":
    print(build_library())
    print(build_torch_ext())
