"""Build the plain-C oracle (attention_ref.c) into oracle/_build/.

TEST INFRASTRUCTURE ONLY: the library is the checker loaded by tests/, never
part of the product path.  The reference itself is pure Python/Triton, so
there is no reference C code to compile into oracle/_ref/.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "attention_ref.c")
OUT_DIR = os.path.join(HERE, "_build")
OUT = os.path.join(OUT_DIR, "liboracle_ref.so")


def build(verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ["gcc", "-O2", "-std=c99", "-shared", "-fPIC", "-Wall", "-Wextra", SRC, "-o", OUT, "-lm"]
    if verbose:
        print("[oracle build]", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return OUT


def load():
    """ctypes handle of the C oracle (built on demand)."""
    import ctypes
    if not os.path.exists(OUT):
        build(verbose=False)
    lib = ctypes.CDLL(OUT)
    dp = ctypes.POINTER(ctypes.c_double)
    ci, cd = ctypes.c_int, ctypes.c_double
    lib.oracle_fwd.restype = ci
    lib.oracle_fwd.argtypes = [dp, dp, dp, ci, ci, ci, ci, cd, ci, dp, dp]
    lib.oracle_bwd.restype = ci
    lib.oracle_bwd.argtypes = [dp, dp, dp, dp, dp, ci, ci, ci, ci, cd, ci, dp, dp, dp, dp]
    return lib


if __name__ == "__main__":
    print(build())
