"""The C-ABI library: loads, exports every declared symbol, and rejects bad
arguments with the documented status codes before touching the GPU.

These run without a GPU: validation happens on the host before any HIP call,
so the pointers below are fake (aligned or deliberately misaligned) integers
that are never dereferenced.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from flash_attn_volta import _capi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "fa_mi355x.h")

P = 0x10000          # fake 16-byte aligned device pointer
BAD = 0x10002        # fake misaligned pointer


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def _st(B, S, H, D):
    """contiguous (B,S,H,D) strides"""
    return (ctypes.c_int64 * 4)(S * H * D, H * D, D, 1)


@pytest.fixture(scope="module")
def lib():
    return _capi.load()


def test_library_exports_every_declared_symbol(lib):
    declared = _declared_functions()
    assert set(declared) == set(_capi.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), f"{name} missing from {_capi.LIB_PATH}"


def test_abi_version(lib):
    assert lib.fa_abi_version() == _capi.ABI_VERSION == 9


def test_noalloc_scratch_size_matches_header():
    m = re.search(r"#define FA_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(HEADER).read())
    assert m and int(m.group(1)) << int(m.group(2)) == _capi.NOALLOC_SCRATCH_BYTES


def test_strerror_covers_every_code(lib):
    codes = [0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11, -12]
    msgs = [lib.fa_strerror(c).decode() for c in codes]
    assert len(set(msgs)) == len(codes)
    assert "unknown" in lib.fa_strerror(-1234).decode()


def _fwd(lib, B=1, S=128, H=2, D=64, q=P, k=P, v=P, o=P, lse=None, st=None, scale=0.125,
         causal=0):
    s = st or _st(B, S, H, D)
    return lib.fa_fwd(q, k, v, o, lse, B, S, H, D, s, s, s, s, scale, causal, None)


def test_fwd_validation(lib):
    assert _fwd(lib, D=48) == _capi.FA_ERR_HEAD_DIM
    assert _fwd(lib, D=16) == _capi.FA_ERR_HEAD_DIM
    assert _fwd(lib, D=256) == _capi.FA_ERR_HEAD_DIM
    assert _fwd(lib, B=0) == _capi.FA_ERR_SHAPE
    assert _fwd(lib, S=-1) == _capi.FA_ERR_SHAPE
    assert _fwd(lib, H=0) == _capi.FA_ERR_SHAPE
    assert _fwd(lib, q=None) == _capi.FA_ERR_NULL_POINTER
    assert _fwd(lib, o=None) == _capi.FA_ERR_NULL_POINTER
    assert _fwd(lib, k=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _fwd(lib, lse=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _fwd(lib, st=(ctypes.c_int64 * 4)(128 * 128, 128, 64, 2)) == _capi.FA_ERR_STRIDE
    assert _fwd(lib, st=(ctypes.c_int64 * 4)(128 * 128, 124, 64, 1)) == _capi.FA_ERR_STRIDE
    assert _fwd(lib, st=(ctypes.c_int64 * 4)(-8, 128, 64, 1)) == _capi.FA_ERR_STRIDE
    assert _fwd(lib, scale=float("nan")) == _capi.FA_ERR_SCALE
    assert _fwd(lib, scale=float("inf")) == _capi.FA_ERR_SCALE
    assert _fwd(lib, S=(1 << 30) + 1) == _capi.FA_ERR_TOO_LARGE


def _bwd(lib, ws=P, ws_bytes=None, lse=P, B=1, S=128, H=2, D=64, scale=0.125, dq=P):
    s = _st(B, S, H, D)
    if ws_bytes is None:
        ws_bytes = lib.fa_bwd_workspace_bytes(B, S, H, D)
    return lib.fa_bwd(P, P, P, P, P, lse, dq, P, P, ws, ws_bytes, B, S, H, D,
                      s, s, s, s, s, s, s, s, scale, 1, None)


def test_workspace_bytes(lib):
    # delta (4 B per row), then the row-group maxima (2 fp32 per 32 rows),
    # each rounded up to 256 B
    assert lib.fa_bwd_workspace_bytes(1, 4096, 16, 64) == 4 * 4096 * 16 + 8 * 128 * 16
    assert lib.fa_bwd_rowmax_bytes(1, 4096, 16) == 8 * 128 * 16
    assert lib.fa_bwd_rowmax_bytes(2, 100, 3) == 256               # 2 x 3 x 4 groups x 8 B -> 256
    assert lib.fa_bwd_rowmax_bytes(1, 33, 40) == 768               # 40 x 2 groups x 8 B = 640 -> 768
    assert lib.fa_bwd_rowmax_bytes(0, 33, 40) == 0
    assert lib.fa_bwd_workspace_bytes(1, 3, 1, 64) == 512          # 256 + 256
    assert lib.fa_bwd_workspace_bytes(1, 3, 1, 48) == 0            # bad D
    assert lib.fa_bwd_workspace_bytes(0, 3, 1, 64) == 0            # bad B


def test_split_workspace_bytes(lib):
    """fa_bwd_gqa_workspace_bytes: the minimum (delta and the row-group
    maxima), plus room for the
    causal key-block (dK/dV) and query-block (dQ) splits only for D = 64 /
    128 causal grids of at most one
    round of resident workgroups (one per CU at D = 128, three at D = 64;
    256 CUs here: without a GPU the count defaults to MI355X's) whose
    longest sweep has at least 32 query tiles (64, or 48 at D = 128, where
    the fused launch could run instead) -- the key-block split only beside the dQ split
    (without it the fused launch runs, unsplit)."""
    mini = lib.fa_bwd_workspace_bytes(1, 4096, 8, 128)
    # (1,4096,8,128) causal: no dQ split (64 blocks x 8 heads is a full
    # round), so the fused D = 128 launch, unsplit: the minimum
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 8, 8, 128, 1) == mini
    # (1,4096,4,128): the dQ grid (64-row blocks x 4 heads, half a round at
    # two per CU) splits its last blocks with more than 64 / 3 = 21 key
    # tiles (43 of 64): 2 x 64 x 128 fp32 each; beside it the key-block
    # split: 32 key blocks x 4 heads, those with > 4 of their 64-query
    # tiles (kt < 30) split, 120 slots of 2 x 2 x 128 x 128 fp32, and 480 B
    # of counters rounded to 512
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 4, 4, 128, 1) == \
        lib.fa_bwd_workspace_bytes(1, 4096, 4, 128) + 512 + 30 * 4 * 2 * 2 * 128 * 128 * 4 + \
        43 * 4 * 2 * 64 * 128 * 4
    # a full round whose block 0 sweeps only 32 tiles: unsplit
    assert lib.fa_bwd_gqa_workspace_bytes(1, 2048, 2048, 16, 16, 128, 1) == \
        lib.fa_bwd_workspace_bytes(1, 2048, 16, 128)
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 8, 8, 128, 0) == mini   # non-causal
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 16, 16, 64, 1) == \
        lib.fa_bwd_workspace_bytes(1, 4096, 16, 64)          # D = 64: 1024 blocks > 3 per CU
    # (1,4096,8,64) causal: no dQ split (64 x 8 blocks are more than half a
    # round), so the fused launch, unsplit: the minimum
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 8, 8, 64, 1) == \
        lib.fa_bwd_workspace_bytes(1, 4096, 8, 64)
    # (1,4096,4,64): the dQ split (64-row blocks x 4 heads, half a round at
    # three per CU; the last 43 with more than 21 key tiles, 2 x 64 x 64
    # fp32 each) and beside it the key-block split (64-key blocks x 4
    # heads, those with more than 21 query tiles, kt < 43: 2 x 2 x 64 x 64
    # fp32 each, 172 counters rounded up to 768 B)
    slots64 = 43 * 4
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 4, 4, 64, 1) == \
        lib.fa_bwd_workspace_bytes(1, 4096, 4, 64) + 768 + slots64 * 2 * 2 * 64 * 64 * 4 + \
        slots64 * 2 * 64 * 64 * 4
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 8, 8, 32, 1) == \
        lib.fa_bwd_workspace_bytes(1, 4096, 8, 32)                                 # D = 32
    assert lib.fa_bwd_gqa_workspace_bytes(1, 4096, 4096, 16, 16, 128, 1) == \
        lib.fa_bwd_workspace_bytes(1, 4096, 16, 128)                               # 512 blocks
    assert lib.fa_bwd_gqa_workspace_bytes(1, 1024, 1024, 16, 16, 128, 1) == \
        lib.fa_bwd_workspace_bytes(1, 1024, 16, 128)                               # 16 tiles
    # grouped heads: tiles count over the 2 query heads of each key head
    # (beside the dQ split, as every D = 128 key split); without the dQ
    # split the fused launch runs unsplit
    assert lib.fa_bwd_gqa_workspace_bytes(1, 3000, 4200, 4, 2, 128, 1) > \
        lib.fa_bwd_workspace_bytes(1, 3000, 4, 128)
    # dQ grids of half a round whose last block sweeps under 64 key tiles:
    # the fused launch, unsplit, in place of the dQ split
    # (under 48 at D = 128)
    for B, S, H, D in ((1, 2048, 8, 64), (2, 2048, 4, 64), (1, 3072, 8, 64),
                       (1, 2048, 8, 128), (1, 2048, 4, 128)):
        assert lib.fa_bwd_gqa_workspace_bytes(B, S, S, H, H, D, 1) == \
            lib.fa_bwd_workspace_bytes(B, S, H, D)
    assert lib.fa_bwd_gqa_workspace_bytes(1, 3072, 3072, 4, 4, 128, 1) > \
        lib.fa_bwd_workspace_bytes(1, 3072, 4, 128)                               # 48 tiles
    assert lib.fa_bwd_gqa_workspace_bytes(1, 2100, 2400, 4, 2, 128, 1) == \
        lib.fa_bwd_workspace_bytes(1, 2100, 4, 128)
    assert lib.fa_bwd_gqa_workspace_bytes(1, 700, 1000, 8, 2, 128, 1) == \
        lib.fa_bwd_workspace_bytes(1, 700, 8, 128)
    assert lib.fa_bwd_gqa_workspace_bytes(1, 700, 1000, 8, 3, 128, 1) == 0       # H % Hk
    assert lib.fa_bwd_gqa_workspace_bytes(1, 700, 1000, 8, 2, 96, 1) == 0        # bad D


def test_bwd_validation(lib):
    assert _bwd(lib, ws=None) == _capi.FA_ERR_WORKSPACE
    assert _bwd(lib, ws_bytes=16) == _capi.FA_ERR_WORKSPACE
    assert _bwd(lib, ws=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _bwd(lib, lse=None) == _capi.FA_ERR_NULL_POINTER
    assert _bwd(lib, lse=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _bwd(lib, dq=None) == _capi.FA_ERR_NULL_POINTER
    assert _bwd(lib, D=96) == _capi.FA_ERR_HEAD_DIM
    assert _bwd(lib, scale=float("nan")) == _capi.FA_ERR_SCALE


def test_preprocess_validation(lib):
    s = _st(1, 64, 1, 64)
    pre = lib.fa_bwd_preprocess
    assert pre(P, P, None, P, 1, 64, 1, 64, s, s, None) == _capi.FA_ERR_NULL_POINTER
    assert pre(P, P, BAD, P, 1, 64, 1, 64, s, s, None) == _capi.FA_ERR_ALIGNMENT
    assert pre(P, P, P, BAD, 1, 64, 1, 64, s, s, None) == _capi.FA_ERR_ALIGNMENT   # row maxima
    assert pre(P, None, P, P, 1, 64, 1, 64, s, s, None) == _capi.FA_ERR_NULL_POINTER
    assert pre(P, P, P, None, 1, 64, 1, 40, s, s, None) == _capi.FA_ERR_HEAD_DIM


def test_standalone_dkdv_needs_row_maxima(lib):
    """fa_bwd_dkdv and fa_bwd_blocks read the pre-pass's row-group maxima
    (their dS bound): NULL or misaligned is refused before any launch."""
    s = _st(1, 64, 1, 64)
    dkdv = lib.fa_bwd_dkdv
    assert dkdv(P, P, P, P, P, P, None, P, P, 1, 64, 1, 64, s, s, s, s, s, s, 0.125, 1,
                None) == _capi.FA_ERR_NULL_POINTER
    assert dkdv(P, P, P, P, P, P, BAD, P, P, 1, 64, 1, 64, s, s, s, s, s, s, 0.125, 1,
                None) == _capi.FA_ERR_ALIGNMENT
    blocks = lib.fa_bwd_blocks
    for causal in (0, 1):
        assert blocks(P, P, P, P, P, P, None, P, P, P, 1, 64, 1, 64, s, s, s, s, s, s, s, 0.125,
                      causal, None) == _capi.FA_ERR_NULL_POINTER


def _fwd_gqa(lib, B=1, Sq=100, Sk=300, H=8, Hk=2, D=64, q=P, k=P, v=P, o=P, lse=None,
             kst=None, scale=0.125, dtype=_capi.FA_DTYPE_F16):
    sq = _st(B, Sq, H, D)
    sk = kst or _st(B, Sk, Hk, D)
    return lib.fa_fwd_gqa(q, k, v, o, lse, B, Sq, Sk, H, Hk, D, sq, sk, sk, sq, scale, 1, dtype,
                          None)


def test_fwd_gqa_validation(lib):
    assert _fwd_gqa(lib, H=8, Hk=3) == _capi.FA_ERR_SHAPE        # H not a multiple of Hk
    assert _fwd_gqa(lib, Hk=0) == _capi.FA_ERR_SHAPE
    assert _fwd_gqa(lib, Sk=0) == _capi.FA_ERR_SHAPE
    assert _fwd_gqa(lib, Sq=0) == _capi.FA_ERR_SHAPE
    assert _fwd_gqa(lib, D=80) == _capi.FA_ERR_HEAD_DIM
    assert _fwd_gqa(lib, v=None) == _capi.FA_ERR_NULL_POINTER
    assert _fwd_gqa(lib, k=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _fwd_gqa(lib, kst=(ctypes.c_int64 * 4)(300 * 128, 128, 60, 1)) == _capi.FA_ERR_STRIDE
    assert _fwd_gqa(lib, scale=float("nan")) == _capi.FA_ERR_SCALE
    assert _fwd_gqa(lib, Sk=(1 << 30) + 1) == _capi.FA_ERR_TOO_LARGE
    assert _fwd_gqa(lib, dtype=2) == _capi.FA_ERR_DTYPE
    assert _fwd_gqa(lib, dtype=-1) == _capi.FA_ERR_DTYPE


def test_bwd_gqa_validation(lib):
    B, Sq, Sk, H, Hk, D = 1, 64, 192, 4, 1, 64
    sq, sk = _st(B, Sq, H, D), _st(B, Sk, Hk, D)
    ws = lib.fa_bwd_workspace_bytes(B, Sq, H, D)

    def call(ws_ptr=P, ws_bytes=ws, Hk_=Hk, dk=P):
        return lib.fa_bwd_gqa(P, P, P, P, P, P, P, dk, P, ws_ptr, ws_bytes, B, Sq, Sk, H, Hk_, D,
                              sq, sq, sk, sk, sq, sq, sk, sk, 0.125, 1, _capi.FA_DTYPE_BF16, None)
    assert call(ws_bytes=ws - 4) == _capi.FA_ERR_WORKSPACE
    assert call(ws_ptr=None) == _capi.FA_ERR_WORKSPACE
    assert call(Hk_=3) == _capi.FA_ERR_SHAPE
    assert call(dk=None) == _capi.FA_ERR_NULL_POINTER
    assert call(dk=BAD) == _capi.FA_ERR_ALIGNMENT


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_capi.LibraryNotBuilt):
        _capi.load(str(tmp_path / "nope.so"))


def _rope_fwd(lib, B=2, S=64, H=4, Hk=2, D=64, q=P, k=P, qo=P, ko=P, cos=P, sin=P, wq=None,
              wk=None, eps=1e-6, qst=None, cs=(64 * 64, 64), dtype=_capi.FA_DTYPE_F16):
    sq = qst or _st(B, S, H, D)
    sk = _st(B, S, Hk, D)
    return lib.fa_rope_qk_fwd(q, k, qo, ko, cos, sin, wq, wk, eps, B, S, H, Hk, D, sq, sk, sq, sk,
                              (ctypes.c_int64 * 2)(*cs), dtype, None)


def test_rope_fwd_validation(lib):
    assert _rope_fwd(lib, D=48) == _capi.FA_ERR_HEAD_DIM
    assert _rope_fwd(lib, D=256) == _capi.FA_ERR_HEAD_DIM
    assert _rope_fwd(lib, B=0) == _capi.FA_ERR_SHAPE
    assert _rope_fwd(lib, Hk=0) == _capi.FA_ERR_SHAPE
    assert _rope_fwd(lib, S=-3) == _capi.FA_ERR_SHAPE
    assert _rope_fwd(lib, dtype=2) == _capi.FA_ERR_DTYPE
    assert _rope_fwd(lib, q=None) == _capi.FA_ERR_NULL_POINTER
    assert _rope_fwd(lib, ko=None) == _capi.FA_ERR_NULL_POINTER
    assert _rope_fwd(lib, sin=None) == _capi.FA_ERR_NULL_POINTER
    assert _rope_fwd(lib, k=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _rope_fwd(lib, cos=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _rope_fwd(lib, wq=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _rope_fwd(lib, cs=(64 * 64, 60)) == _capi.FA_ERR_STRIDE
    assert _rope_fwd(lib, cs=(-8, 64)) == _capi.FA_ERR_STRIDE
    assert _rope_fwd(lib, qst=(ctypes.c_int64 * 4)(64 * 256, 256, 64, 2)) == _capi.FA_ERR_STRIDE
    assert _rope_fwd(lib, wq=P, eps=-1e-6) == _capi.FA_ERR_EPS
    assert _rope_fwd(lib, wk=P, eps=float("nan")) == _capi.FA_ERR_EPS
    assert _rope_fwd(lib, wk=P, eps=float("inf")) == _capi.FA_ERR_EPS
    assert _rope_fwd(lib, B=1, S=1 << 20, H=4096, Hk=8) == _capi.FA_ERR_TOO_LARGE   # 2^32 rows


def test_rope_bwd_validation(lib):
    B, S, H, Hk, D = 1, 128, 8, 2, 128
    sq, sk = _st(B, S, H, D), _st(B, S, Hk, D)
    cs = (ctypes.c_int64 * 2)(0, D)
    ws = lib.fa_rope_qk_workspace_bytes(B, S, H, Hk, D)
    assert ws > 0 and ws % 16 == 0
    assert lib.fa_rope_qk_workspace_bytes(B, S, H, Hk, 96) == 0
    assert lib.fa_rope_qk_workspace_bytes(0, S, H, Hk, D) == 0

    def call(q=P, wq=P, dwq=P, ws_ptr=P, ws_bytes=ws, dq=P, eps=1e-6):
        return lib.fa_rope_qk_bwd(P, P, q, P, P, P, wq, None, eps, dq, P, dwq, None, ws_ptr,
                                  ws_bytes, B, S, H, Hk, D, sq, sk, sq, sk, sq, sk, cs,
                                  _capi.FA_DTYPE_BF16, None)
    assert call(ws_bytes=ws - 4) == _capi.FA_ERR_WORKSPACE
    assert call(ws_ptr=None) == _capi.FA_ERR_WORKSPACE
    assert call(ws_ptr=BAD) == _capi.FA_ERR_ALIGNMENT
    assert call(q=None) == _capi.FA_ERR_NULL_POINTER        # a normed side needs its input
    assert call(dwq=None) == _capi.FA_ERR_NULL_POINTER      # ... and its weight-gradient output
    assert call(dq=None) == _capi.FA_ERR_NULL_POINTER
    assert call(dq=BAD) == _capi.FA_ERR_ALIGNMENT
    assert call(eps=-1.0) == _capi.FA_ERR_EPS


def test_fwd_workspace_plan_and_validation(lib):
    """fa_fwd_ws: the workspace query (256 compute units assumed on the CPU)
    is the split-KV size for decode shapes, the balanced causal size for
    square causal grids of at least 32 tiles per head and at most half a
    tile per CU (one from 48 tiles per head, 1.75 from 64),
    0 otherwise; a call that would use a workspace rejects a misaligned one
    before any HIP call."""
    ws = lib.fa_fwd_workspace_bytes
    kv = lib.fa_fwd_splitkv_workspace_bytes
    assert ws(1, 1, 4096, 32, 8, 128, 1) == kv(1, 1, 4096, 32, 8, 128) > 0   # decode
    n = ws(1, 4096, 4096, 4, 4, 128, 1)          # 64 tiles x 4 heads: one per CU
    rows = 1 * 4 * (4096 // 64 // 2) * 64        # (b, h, pair, row) of the split tiles
    assert n % 256 == 0 and n >= 2 * rows * (128 + 1) * 4
    assert ws(1, 4096, 4096, 4, 2, 128, 1) == n  # grouped heads: same grid
    assert ws(1, 4096, 4096, 4, 4, 128, 0) == 0  # not causal
    assert ws(1, 4096, 4096, 8, 8, 128, 1) == 0  # two tiles per CU (config C4b)
    assert ws(1, 4096, 4096, 6, 6, 128, 1) > n    # 1.5 tiles per CU
    assert ws(1, 4096, 4096, 7, 7, 128, 1) > n    # 1.75
    assert ws(1, 8192, 8192, 4, 4, 128, 1) == 0   # 2
    assert ws(1, 2048, 2048, 4, 4, 128, 1) > 0   # 32 tiles, half a tile per CU
    assert ws(1, 2048, 2048, 8, 8, 128, 1) == 0  # 32 tiles, one per CU
    assert ws(1, 1984, 1984, 2, 2, 128, 1) == 0  # 31 tiles per head: too few
    assert ws(1, 3072, 3072, 4, 4, 128, 1) > 0   # 48 tiles, one per CU
    assert ws(1, 3072, 3072, 6, 6, 128, 1) == 0  # 48 tiles, 1.125 per CU
    assert ws(1, 4000, 4096, 4, 4, 128, 1) == 0  # Sq != Sk
    assert ws(1, 4096, 4096, 4, 3, 128, 1) == 0  # invalid (H % Hk)
    st = _st(1, 4096, 4, 128)
    assert lib.fa_fwd_ws(P, P, P, P, None, BAD, n, 1, 4096, 4096, 4, 4, 128, st, st, st, st,
                         0.1, 1, _capi.FA_DTYPE_F16, None) == _capi.FA_ERR_ALIGNMENT
    assert lib.fa_fwd_ws(None, P, P, P, None, P, n, 1, 4096, 4096, 4, 4, 128, st, st, st, st,
                         0.1, 1, _capi.FA_DTYPE_F16, None) == _capi.FA_ERR_NULL_POINTER
    assert lib.fa_fwd_ws(P, P, P, P, None, P, n, 1, 4096, 4096, 4, 4, 96, st, st, st, st,
                         0.1, 1, _capi.FA_DTYPE_F16, None) == _capi.FA_ERR_HEAD_DIM


def test_splitkv_plan_and_validation(lib):
    """fa_fwd_splitkv: the workspace query (on the CPU the library assumes
    MI355X's 256 compute units) is non-zero exactly for decode-like sizes,
    and a splitting call rejects a missing or short workspace before any
    HIP call."""
    ws = lib.fa_fwd_splitkv_workspace_bytes
    assert ws(1, 1, 4096, 32, 8, 128) > 0            # decode, GQA group of 4
    assert ws(1, 8, 4096, 64, 8, 128) > 0            # 8 query rows x group of 8 = 64
    assert ws(1, 9, 4096, 64, 8, 128) == 0           # 72 rows: no single tile
    assert ws(1, 4096, 4096, 16, 16, 64) == 0        # prefill fills the GPU
    assert ws(1, 1, 128, 32, 8, 128) == 0            # too few keys
    assert ws(64, 1, 4096, 32, 32, 128) == 0         # regular grid already full
    assert ws(1, 1, 4096, 30, 8, 128) == 0           # invalid (H % Hk)
    n = ws(1, 1, 4096, 32, 8, 128)
    assert n % 256 == 0 and n >= 2 * 32 * (128 + 1) * 4
    sq, sk = _st(1, 1, 32, 128), _st(1, 4096, 8, 128)

    def call(w=P, nb=n, Sk=4096):
        return lib.fa_fwd_splitkv(P, P, P, P, None, w, nb, 1, 1, Sk, 32, 8, 128, sq, sk, sk, sq,
                                  0.1, 1, _capi.FA_DTYPE_F16, None)
    assert call(w=None) == _capi.FA_ERR_WORKSPACE
    assert call(nb=n - 16) == _capi.FA_ERR_WORKSPACE
    assert call(w=BAD) == _capi.FA_ERR_ALIGNMENT
    assert lib.fa_fwd_splitkv(P, P, P, P, None, P, n, 1, 1, 4096, 32, 8, 96, sq, sk, sk, sq,
                              0.1, 1, 0, None) == _capi.FA_ERR_HEAD_DIM


def test_sequence_stride_bound_for_32bit_tile_offsets(lib):
    """Inside a tile the kernels address up to 128 rows of a head with 32-bit
    byte offsets (row * seq_stride * 2): a sequence stride that would carry
    127 rows past 2^31 bytes is FA_ERR_TOO_LARGE, not a silent wrap.  The
    bound is checked on every attention tensor, input or output, and is
    moot for a single row (its stride addresses nothing).  Calls meant to
    pass the stride checks carry a NaN scale, which is checked after every
    tensor, so they return FA_ERR_SCALE and launch nothing (the pointers
    are fake)."""
    B, S, H, D = 1, 256, 1, 64
    nan = float("nan")
    ok = (2**31 - 1 - 2 * D) // 254 // 8 * 8          # largest multiple of 8 that fits
    big = ok + 8

    def st(seq):
        return (ctypes.c_int64 * 4)(seq * S, seq, D, 1)
    good, bad, base = st(ok), st(big), _st(B, S, H, D)
    f = lib.fa_fwd
    assert f(P, P, P, P, None, B, S, H, D, good, good, good, good, nan, 0, None) == \
        _capi.FA_ERR_SCALE
    for args in ((bad, base, base, base), (base, bad, base, base), (base, base, bad, base),
                 (base, base, base, bad)):
        assert f(P, P, P, P, None, B, S, H, D, *args, 0.1, 0, None) == _capi.FA_ERR_TOO_LARGE
    # one query row: its stride is never used
    one = (ctypes.c_int64 * 4)(big, big, D, 1)
    assert lib.fa_fwd_gqa(P, P, P, P, None, B, 1, S, H, H, D, one, base, base, _st(B, 1, H, D),
                          nan, 0, _capi.FA_DTYPE_F16, None) == _capi.FA_ERR_SCALE
    # the backward checks its tensors the same way
    sq = _st(B, S, H, D)
    ws = lib.fa_bwd_workspace_bytes(B, S, H, D)
    assert lib.fa_bwd(P, P, P, P, P, P, P, P, P, P, ws, B, S, H, D, sq, sq, bad, sq, sq, sq, sq,
                      sq, 0.1, 1, None) == _capi.FA_ERR_TOO_LARGE


def test_sequence_stride_bound_is_exact():
    """The bound is the exact one the kernels need: 127 rows of the largest
    accepted stride plus one D-row end below 2^31 bytes; eight more
    elements do not."""
    D = 64
    ok = (2**31 - 1 - 2 * D) // 254 // 8 * 8
    assert 127 * ok * 2 + 2 * D <= 2**31 - 1 < 127 * (ok + 8) * 2 + 2 * D


def test_output_rows_must_not_overlap(lib):
    """Written tensors (o, dq, dk, dv, rope outputs) whose (b, s, h) rows
    share elements -- a zero stride on a dimension of size > 1, or a stride
    below the extent of the rows nested inside it -- are FA_ERR_STRIDE:
    workgroups would store the same bytes in a schedule-dependent order.
    Inputs may overlap (broadcast reads are fine), size-1 dimensions may
    have any stride, and sliced views pass.  Calls meant to pass carry a NaN
    scale (checked after every tensor): FA_ERR_SCALE, nothing launched."""
    B, S, H, D = 2, 64, 4, 64
    nan = float("nan")
    base = _st(B, S, H, D)
    f = lib.fa_fwd
    for o_st in ((0, H * D, D, 1),              # two batches on one output
                 (S * H * D, 0, D, 1),          # every position on one row
                 (S * H * D, H * D, 0, 1),      # heads collapse
                 (S * H * D, 64, D, 1)):        # seq stride inside a position's heads
        o = (ctypes.c_int64 * 4)(*o_st)
        assert f(P, P, P, P, None, B, S, H, D, base, base, base, o, 0.1, 0, None) == \
            _capi.FA_ERR_STRIDE, o_st
    # broadcast input (zero batch stride on k and v): not an output
    kb = (ctypes.c_int64 * 4)(0, H * D, D, 1)
    assert f(P, P, P, P, None, B, S, H, D, base, kb, kb, base, nan, 0, None) == _capi.FA_ERR_SCALE
    # a (B,S,H,D) output that is a slice of a (B,S,2H,D) buffer, and the
    # (B,H,S,D).transpose(1,2) layout, are disjoint
    for o_st in ((S * 2 * H * D, 2 * H * D, D, 1), (H * S * D, D, S * D, 1)):
        o = (ctypes.c_int64 * 4)(*o_st)
        assert f(P, P, P, P, None, B, S, H, D, base, base, base, o, nan, 0, None) == \
            _capi.FA_ERR_SCALE
    # size-1 dims may carry any stride, zero included
    o1 = (ctypes.c_int64 * 4)(0, 0, D, 1)
    b1 = _st(1, 1, H, D)
    assert f(P, P, P, P, None, 1, 1, H, D, b1, b1, b1, o1, nan, 0, None) == _capi.FA_ERR_SCALE
    # backward outputs and the rope outputs are checked the same way
    ws = lib.fa_bwd_workspace_bytes(B, S, H, D)
    z = (ctypes.c_int64 * 4)(0, H * D, D, 1)
    assert lib.fa_bwd(P, P, P, P, P, P, P, P, P, P, ws, B, S, H, D, base, base, base, base, base,
                      base, base, z, 0.1, 1, None) == _capi.FA_ERR_STRIDE
    assert lib.fa_bwd(P, P, P, P, P, P, P, P, P, P, ws, B, S, H, D, base, base, base, base, base,
                      z, base, base, 0.1, 1, None) == _capi.FA_ERR_STRIDE
    cs = (ctypes.c_int64 * 2)(0, D)
    assert lib.fa_rope_qk_fwd(P, P, P, P, P, P, None, None, 0.0, B, S, H, H, D, base, base, z,
                              base, cs, _capi.FA_DTYPE_F16, None) == _capi.FA_ERR_STRIDE


def _bwd_noalloc(lib, B=1, Sq=128, Sk=128, H=2, Hk=2, D=64, lse=P, dq=P, dk_st=None,
                 scale=0.125, dtype=_capi.FA_DTYPE_F16):
    sq, sk = _st(B, Sq, H, D), _st(B, Sk, Hk, D)
    return lib.fa_bwd_gqa_noalloc(P, P, P, P, P, lse, dq, P, P, B, Sq, Sk, H, Hk, D,
                                  sq, sq, sk, sk, sq, sq, dk_st or sk, sk, scale, 1, dtype, None)


def test_noalloc_validation_before_any_hip_call(lib):
    """fa_bwd_gqa_noalloc validates everything fa_bwd_gqa does (but the
    workspace, which it does not take) and rejects a problem whose delta
    (4 * B * H * Sq bytes) exceeds the static scratch buffer with
    FA_ERR_SCRATCH -- all before any HIP call, so on a GPU-less machine the
    codes come back exactly (and on a GPU box nothing launches: every call
    here is invalid)."""
    assert _bwd_noalloc(lib, D=96) == _capi.FA_ERR_HEAD_DIM
    assert _bwd_noalloc(lib, Hk=3) == _capi.FA_ERR_SHAPE
    assert _bwd_noalloc(lib, lse=None) == _capi.FA_ERR_NULL_POINTER
    assert _bwd_noalloc(lib, lse=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _bwd_noalloc(lib, dq=BAD) == _capi.FA_ERR_ALIGNMENT
    assert _bwd_noalloc(lib, scale=float("inf")) == _capi.FA_ERR_SCALE
    assert _bwd_noalloc(lib, dtype=3) == _capi.FA_ERR_DTYPE
    assert _bwd_noalloc(lib, dk_st=(ctypes.c_int64 * 4)(0, 0, 64, 1)) == _capi.FA_ERR_STRIDE
    # one query row more than the scratch holds: 64 heads x Sq rows x 4 bytes
    rows = _capi.NOALLOC_SCRATCH_BYTES // 4
    assert _bwd_noalloc(lib, B=1, Sq=rows // 64 + 1, Sk=128, H=64, Hk=64) == _capi.FA_ERR_SCRATCH
    assert lib.fa_strerror(_capi.FA_ERR_SCRATCH).decode().startswith("fa_bwd_gqa_noalloc")


def test_torch_node_module_loads():
    """The C++ autograd node (_fa_torch.so, built on the C ABI) imports on a
    machine without a GPU and rejects a malformed plan."""
    import pytest
    try:
        from flash_attn_volta import _fa_torch
    except ImportError as e:
        pytest.fail(f"_fa_torch is not built or does not load: {e}")
    assert _fa_torch.PLAN_INTS == 36
    with pytest.raises(RuntimeError, match="expected 36 integers"):
        _fa_torch.make_plan([1, 2, 3], 0.125)
    with pytest.raises(RuntimeError, match="unknown plan handle"):
        import torch
        t = torch.zeros(8)
        _fa_torch.attn(12345, t, t, t, True)


_STUB_LIB = r"""
#include <stddef.h>
int fa_abi_version(void) { return %d; }
const char *fa_strerror(int s) { (void)s; return "stub"; }
int fa_fwd(void) { return -9; }
int fa_fwd_gqa(void) { return -9; }
int fa_fwd_ws(void) { return -9; }
int fa_bwd(void) { return -9; }
int fa_bwd_gqa(void) { return -9; }
"""


def test_torch_node_refuses_a_library_of_another_abi(tmp_path):
    """_fa_torch calls the library with the argument lists of the header it
    was compiled against, so it must not load beside a libfa_mi355x.so of
    another ABI version (the two are built separately).  A copy of the built
    module next to a stub library that reports another version (rpath
    $ORIGIN picks the stub) raises ImportError on import (pybind11 chains
    the module's own message as its cause) -- the error that autograd.py
    turns into the Python autograd path -- while the real pair imports."""
    import shutil
    import subprocess
    import sys

    pkg = os.path.dirname(os.path.abspath(_capi.__file__))
    ext = os.path.join(pkg, "_fa_torch.so")
    if not os.path.exists(ext):
        pytest.skip("_fa_torch.so is not built")
    src = tmp_path / "stub.c"
    src.write_text(_STUB_LIB % (_capi.ABI_VERSION + 1000))
    subprocess.run(["gcc", "-shared", "-fPIC", str(src), "-o", str(tmp_path / "libfa_mi355x.so")],
                   check=True)
    shutil.copy(ext, tmp_path / "_fa_torch.so")
    probe = (
        "import importlib.util, sys, torch\n"
        "spec = importlib.util.spec_from_file_location('_fa_torch', sys.argv[1])\n"
        "m = importlib.util.module_from_spec(spec)\n"
        "try:\n"
        "    spec.loader.exec_module(m)\n"
        "except ImportError as e:\n"
        "    print('IMPORT_ERROR', e, e.__cause__)\n"
        "else:\n"
        "    print('LOADED', m.PLAN_INTS)\n")
    bad = subprocess.run([sys.executable, "-c", probe, str(tmp_path / "_fa_torch.so")],
                         capture_output=True, text=True, timeout=300)
    assert "IMPORT_ERROR" in bad.stdout, bad.stdout + bad.stderr
    assert f"ABI {_capi.ABI_VERSION}" in bad.stdout and "rebuild" in bad.stdout
    good = subprocess.run([sys.executable, "-c", probe, ext], capture_output=True, text=True,
                          timeout=300)
    assert "LOADED 36" in good.stdout, good.stdout + good.stderr
