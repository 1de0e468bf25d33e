"""ctypes binding of the gfx950 FlashAttention C ABI (include/fa_mi355x.h).

The shared library ``libfa_mi355x.so`` is built in-tree next to this file by
``flash_attn_volta.build.build_library()``.  There is no fallback: if the
library is missing every compute entry point raises, so a run can never
silently take a CPU or eager-PyTorch path.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libfa_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

ABI_VERSION = 9

# status codes (enum fa_status)
FA_OK = 0
FA_ERR_NULL_POINTER = -1
FA_ERR_HEAD_DIM = -2
FA_ERR_SHAPE = -3
FA_ERR_STRIDE = -4
FA_ERR_ALIGNMENT = -5
FA_ERR_SCALE = -6
FA_ERR_WORKSPACE = -7
FA_ERR_TOO_LARGE = -8
FA_ERR_LAUNCH = -9
FA_ERR_DTYPE = -10
FA_ERR_EPS = -11
FA_ERR_SCRATCH = -12

# bytes of the static device buffer fa_bwd_gqa_noalloc uses as its workspace
NOALLOC_SCRATCH_BYTES = 64 << 20

# element types (enum fa_dtype)
FA_DTYPE_F16 = 0
FA_DTYPE_BF16 = 1

# Every symbol include/fa_mi355x.h declares.
EXPORTED_SYMBOLS = (
    "fa_abi_version",
    "fa_strerror",
    "fa_fwd",
    "fa_fwd_gqa",
    "fa_fwd_splitkv",
    "fa_fwd_splitkv_workspace_bytes",
    "fa_fwd_ws",
    "fa_fwd_workspace_bytes",
    "fa_bwd_preprocess",
    "fa_bwd_rowmax_bytes",
    "fa_bwd_workspace_bytes",
    "fa_bwd_gqa_workspace_bytes",
    "fa_bwd",
    "fa_bwd_gqa",
    "fa_bwd_gqa_noalloc",
    "fa_bwd_dkdv",
    "fa_bwd_dq",
    "fa_bwd_blocks",
    "fa_rope_qk_fwd",
    "fa_rope_qk_workspace_bytes",
    "fa_rope_qk_bwd",
)

_lock = threading.Lock()
_lib = None

_i64x4 = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_ci = ctypes.c_int


class LibraryNotBuilt(RuntimeError):
    pass


class FlashAttnError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {strerror(status)} (status {status})")


def _declare(lib):
    lib.fa_abi_version.restype = _ci
    lib.fa_abi_version.argtypes = []
    lib.fa_strerror.restype = ctypes.c_char_p
    lib.fa_strerror.argtypes = [_ci]
    lib.fa_fwd.restype = _ci
    lib.fa_fwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci,
                           _i64x4, _i64x4, _i64x4, _i64x4,
                           ctypes.c_float, _ci, _vp]
    lib.fa_fwd_gqa.restype = _ci
    lib.fa_fwd_gqa.argtypes = [_vp, _vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci, _ci, _ci,
                               _i64x4, _i64x4, _i64x4, _i64x4,
                               ctypes.c_float, _ci, _ci, _vp]
    lib.fa_fwd_splitkv.restype = _ci
    lib.fa_fwd_splitkv.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                   _ci, _ci, _ci, _ci, _ci, _ci,
                                   _i64x4, _i64x4, _i64x4, _i64x4,
                                   ctypes.c_float, _ci, _ci, _vp]
    lib.fa_fwd_splitkv_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_fwd_splitkv_workspace_bytes.argtypes = [_ci, _ci, _ci, _ci, _ci, _ci]
    lib.fa_fwd_ws.restype = _ci
    lib.fa_fwd_ws.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                              _ci, _ci, _ci, _ci, _ci, _ci,
                              _i64x4, _i64x4, _i64x4, _i64x4,
                              ctypes.c_float, _ci, _ci, _vp]
    lib.fa_fwd_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_fwd_workspace_bytes.argtypes = [_ci, _ci, _ci, _ci, _ci, _ci, _ci]
    lib.fa_bwd_preprocess.restype = _ci
    lib.fa_bwd_preprocess.argtypes = [_vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci, _i64x4, _i64x4, _vp]
    lib.fa_bwd_rowmax_bytes.restype = ctypes.c_size_t
    lib.fa_bwd_rowmax_bytes.argtypes = [_ci, _ci, _ci]
    lib.fa_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_bwd_workspace_bytes.argtypes = [_ci, _ci, _ci, _ci]
    lib.fa_bwd_gqa_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_bwd_gqa_workspace_bytes.argtypes = [_ci, _ci, _ci, _ci, _ci, _ci, _ci]
    lib.fa_bwd.restype = _ci
    lib.fa_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp,
                           _vp, _vp, _vp,
                           _vp, ctypes.c_size_t,
                           _ci, _ci, _ci, _ci,
                           _i64x4, _i64x4, _i64x4, _i64x4,
                           _i64x4, _i64x4, _i64x4, _i64x4,
                           ctypes.c_float, _ci, _vp]
    lib.fa_bwd_gqa.restype = _ci
    lib.fa_bwd_gqa.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp,
                               _vp, _vp, _vp,
                               _vp, ctypes.c_size_t,
                               _ci, _ci, _ci, _ci, _ci, _ci,
                               _i64x4, _i64x4, _i64x4, _i64x4,
                               _i64x4, _i64x4, _i64x4, _i64x4,
                               ctypes.c_float, _ci, _ci, _vp]
    lib.fa_bwd_gqa_noalloc.restype = _ci
    lib.fa_bwd_gqa_noalloc.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _vp,
                                       _ci, _ci, _ci, _ci, _ci, _ci,
                                       _i64x4, _i64x4, _i64x4, _i64x4,
                                       _i64x4, _i64x4, _i64x4, _i64x4,
                                       ctypes.c_float, _ci, _ci, _vp]
    lib.fa_bwd_dkdv.restype = _ci
    lib.fa_bwd_dkdv.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _ci, _ci, _ci, _ci,
                                _i64x4, _i64x4, _i64x4, _i64x4, _i64x4, _i64x4,
                                ctypes.c_float, _ci, _vp]
    lib.fa_bwd_dq.restype = _ci
    lib.fa_bwd_dq.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp,
                              _ci, _ci, _ci, _ci,
                              _i64x4, _i64x4, _i64x4, _i64x4, _i64x4,
                              ctypes.c_float, _ci, _vp]
    lib.fa_bwd_blocks.restype = _ci
    lib.fa_bwd_blocks.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _ci, _ci, _ci, _ci,
                                  _i64x4, _i64x4, _i64x4, _i64x4, _i64x4, _i64x4, _i64x4,
                                  ctypes.c_float, _ci, _vp]
    _i64x2 = ctypes.POINTER(ctypes.c_int64)
    lib.fa_rope_qk_fwd.restype = _ci
    lib.fa_rope_qk_fwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                   _ci, _ci, _ci, _ci, _ci,
                                   _i64x4, _i64x4, _i64x4, _i64x4, _i64x2, _ci, _vp]
    lib.fa_rope_qk_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_rope_qk_workspace_bytes.argtypes = [_ci, _ci, _ci, _ci, _ci]
    lib.fa_rope_qk_bwd.restype = _ci
    lib.fa_rope_qk_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                   _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                   _ci, _ci, _ci, _ci, _ci,
                                   _i64x4, _i64x4, _i64x4, _i64x4, _i64x4, _i64x4,
                                   _i64x2, _ci, _vp]


def load(path: str | None = None):
    """Load (once) and return the ctypes handle of the C-ABI library."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise LibraryNotBuilt(
                f"{p} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(or flash_attn_volta.build.build_library()) first. There is no fallback path.")
        lib = ctypes.CDLL(p)
        _declare(lib)
        v = lib.fa_abi_version()
        if v != ABI_VERSION:
            raise LibraryNotBuilt(f"{p} has ABI version {v}, expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def strerror(status: int) -> str:
    try:
        return load().fa_strerror(int(status)).decode()
    except LibraryNotBuilt:
        return f"status {status}"


def strides4(t) -> ctypes.Array:
    """(b, s, h, d) element strides of a 4-D tensor as a C int64[4]."""
    return (ctypes.c_int64 * 4)(*[int(x) for x in t.stride()])


def check(status: int, where: str) -> None:
    if status != FA_OK:
        raise FlashAttnError(status, where)
