"""Forward attention over (B, S, H, D) fp16 tensors on an MI355X.

Drop-in for the reference's ``flash_attn_forward`` / ``flash_attn_volta``
(flash_attn_volta/triton_fa.py:291-401): same signature, defaults, return
arity, layouts and the +inf LSE rule for rows that see no key
(triton_fa.py:152-157).  The work is one launch of the hand-written gfx950
kernel behind ``fa_fwd`` (include/fa_mi355x.h); the (B, S, H, D) strides go
straight to the kernel, so there are no permute copies, and D = 32 / 64 / 128
run natively with no padding.  D = 16, which the reference also accepts
(triton_fa.py:317), is zero-padded to 32 here (an on-device copy; the padded
columns contribute exactly zero to every dot product).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _capi

SUPPORTED_HEAD_DIMS = (16, 32, 64, 128)
NATIVE_HEAD_DIMS = (32, 64, 128)


class FlashAttnArgumentError(AssertionError, ValueError):
    """Invalid arguments.  Subclasses AssertionError, which is what the
    reference raises for the same checks (triton_fa.py:313-317), and
    ValueError."""


def _require(cond: bool, msg) -> None:
    """Raise FlashAttnArgumentError(msg) unless `cond`.  `msg` is a string,
    or a callable returning one: messages that format tensor shapes are
    passed as lambdas so that a passing check costs no string formatting
    (a few microseconds per call on the launch path)."""
    if not cond:
        raise FlashAttnArgumentError(msg() if callable(msg) else msg)


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` if the kernel can read it in place (unit D stride,
    16-byte aligned base, other strides multiples of 8 elements), else a
    contiguous copy."""
    if t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t            # D is a multiple of 8, so every stride is too
    ok = t.stride(3) == 1 and t.data_ptr() % 16 == 0
    if ok:
        for dim in range(3):
            if t.size(dim) != 1 and (t.stride(dim) % 8 != 0 or t.stride(dim) < 0):
                ok = False
                break
    return t if ok else t.contiguous()


_STRIDES = {}


def kernel_strides(t: torch.Tensor):
    """C int64[4] strides, with 0 for size-1 dims (their stride is never
    used).  The ctypes arrays are cached per layout: they are read-only."""
    key = (t.shape, t.stride())
    arr = _STRIDES.get(key)
    if arr is None:
        st = [0 if t.size(i) == 1 and i < 3 else int(t.stride(i)) for i in range(4)]
        arr = (ctypes.c_int64 * 4)(*st)
        if len(_STRIDES) > 4096:
            _STRIDES.clear()
        _STRIDES[key] = arr
    return arr


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    """hipStream_t of the device's current stream (the raw query skips
    building a Stream object; same value)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


class _on_device:
    """Make `device` current for the duration of a launch, skipping the
    context switch in the common case where it already is."""
    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        self.idx = device.index

    def __enter__(self):
        self.prev = torch.cuda.current_device()
        if self.prev != self.idx:
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev != self.idx:
            torch.cuda.set_device(self.prev)
        return False


def _pad_d(t: torch.Tensor, d_to: int) -> torch.Tensor:
    return torch.nn.functional.pad(t, (0, d_to - t.size(-1)))


def flash_attn_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float | None = None,
    return_softmax_lse: bool = False,
):
    """FlashAttention forward: fp16 in/out, fp32 accumulation.

    Args:
        q, k, v: (B, N, H, D) fp16 on the GPU. D in {16, 32, 64, 128}.
        causal: apply the lower-triangular mask.
        sm_scale: softmax scale (default 1/sqrt(D)).
        return_softmax_lse: also return the per-row natural-log LSE.

    Returns:
        out (B, N, H, D) fp16 contiguous, and, if ``return_softmax_lse``,
        lse (B, H, N) fp32 contiguous (+inf for a row that sees no key).
    """
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "tensors must be on CUDA")
    _require(q.dtype == torch.float16 == k.dtype == v.dtype, "fp16 only")
    _require(q.shape == k.shape == v.shape, lambda: f"qkv shape mismatch {q.shape} {k.shape} {v.shape}")
    _require(q.dim() == 4, lambda: f"expected (B, N, H, D) tensors, got {tuple(q.shape)}")
    _require(q.device == k.device == v.device, "q, k, v must be on one device")
    B, N, H, D = q.shape
    _require(D in SUPPORTED_HEAD_DIMS, lambda: f"unsupported head_dim {D} (allowed: 16,32,64,128)")

    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)

    return _forward(q, k, v, causal, sm_scale, return_softmax_lse, gqa=False)


def _forward(q, k, v, causal, sm_scale, return_softmax_lse, gqa):
    D = q.shape[-1]
    if D not in NATIVE_HEAD_DIMS:
        out, lse = _run_fwd(_pad_d(q, 32), _pad_d(k, 32), _pad_d(v, 32), causal, sm_scale,
                            return_softmax_lse, gqa)
        out = out[..., :D].contiguous()
    else:
        out, lse = _run_fwd(q, k, v, causal, sm_scale, return_softmax_lse, gqa)
    if return_softmax_lse:
        return out, lse
    return out


_DTYPES = {torch.float16: _capi.FA_DTYPE_F16, torch.bfloat16: _capi.FA_DTYPE_BF16}


def _run_fwd(q, k, v, causal, sm_scale, write_lse, gqa):
    lib = _capi.load()
    B, N, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    out = torch.empty((B, N, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, N), dtype=torch.float32, device=q.device) if write_lse else None
    if out.numel() == 0 or Sk == 0:
        # no query, or no key: every row sees nothing (O = 0, LSE = +inf)
        out.zero_()
        if lse is not None:
            lse.fill_(float("inf"))
        return out, lse
    st = (kernel_strides(q), kernel_strides(k), kernel_strides(v), kernel_strides(out))
    lse_ptr = lse.data_ptr() if lse is not None else None
    with _on_device(q.device):
        ws = _splitkv_workspace(lib, B, N, Sk, H, Hk, D, q.device) if gqa else None
        if ws is not None:
            # short query block against long keys (decode): split the keys
            rc = lib.fa_fwd_splitkv(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                    lse_ptr, ws.data_ptr(), ws.numel(), B, N, Sk, H, Hk, D, *st,
                                    float(sm_scale), int(bool(causal)), _DTYPES[q.dtype],
                                    _stream_ptr(q.device))
            _capi.check(rc, "fa_fwd_splitkv")
            return out, lse
        if gqa:
            rc = lib.fa_fwd_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse_ptr,
                                B, N, Sk, H, Hk, D, *st,
                                float(sm_scale), int(bool(causal)), _DTYPES[q.dtype],
                                _stream_ptr(q.device))
        else:
            rc = lib.fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse_ptr,
                            B, N, H, D, *st,
                            float(sm_scale), int(bool(causal)), _stream_ptr(q.device))
    _capi.check(rc, "fa_fwd_gqa" if gqa else "fa_fwd")
    return out, lse


_SPLITKV_BYTES = {}


def _splitkv_workspace(lib, B, Sq, Sk, H, Hk, D, device):
    """Workspace tensor for fa_fwd_splitkv when the library would split the
    keys for these sizes on this device (decode-like shapes), else None.
    Only short query blocks can qualify, so longer ones skip the query."""
    if (H // Hk) * Sq > 64:
        return None
    key = (B, Sq, Sk, H, Hk, D, device.index)
    nbytes = _SPLITKV_BYTES.get(key)
    if nbytes is None:
        nbytes = _SPLITKV_BYTES[key] = int(lib.fa_fwd_splitkv_workspace_bytes(B, Sq, Sk, H, Hk, D))
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _check_gqa(q, k, v):
    """Shape rules of the grouped-query entry points: q (B, Sq, H, D),
    k and v (B, Sk, Hk, D) with H a multiple of Hk."""
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4,
             f"expected 4-D (B, N, H, D) tensors, got {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    _require(k.shape == v.shape, lambda: f"k and v shapes differ: {tuple(k.shape)} {tuple(v.shape)}")
    _require(q.shape[0] == k.shape[0], lambda: f"batch mismatch {q.shape[0]} vs {k.shape[0]}")
    _require(q.shape[3] == k.shape[3], lambda: f"head_dim mismatch {q.shape[3]} vs {k.shape[3]}")
    H, Hk = q.shape[2], k.shape[2]
    _require(Hk > 0 and H % Hk == 0,
             f"query heads ({H}) must be a multiple of key/value heads ({Hk})")


def flash_attn_forward_gqa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float | None = None,
    return_softmax_lse: bool = False,
):
    """Grouped-query / multi-query attention forward with independent query
    and key lengths (no counterpart in the reference; it removes the
    repeat_kv copy and the KV-cache fallback of the reference's HF patch,
    flash_attn_volta/patch_hf.py:145-162, 186-188).

    Args:
        q: (B, Sq, H, D) on the GPU; k, v: (B, Sk, Hk, D) with H a multiple
            of Hk.  Query head h uses key/value head h // (H // Hk), the head
            order of HuggingFace's ``repeat_kv``.  fp16 or bf16 (all three
            alike; the output has the same dtype, accumulation is fp32).
        causal: bottom-right aligned mask: query i sees key j iff
            j <= i + Sk - Sq (a query with no visible key gets 0 output and
            +inf LSE).  With Sq == Sk it is the usual causal mask.
        sm_scale, return_softmax_lse: as in ``flash_attn_forward``.
    """
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "tensors must be on CUDA")
    _require(q.dtype in _DTYPES and q.dtype == k.dtype == v.dtype,
             f"fp16 or bf16 only, all alike (got {q.dtype}, {k.dtype}, {v.dtype})")
    _require(q.device == k.device == v.device, "q, k, v must be on one device")
    _check_gqa(q, k, v)
    D = q.shape[3]
    _require(D in SUPPORTED_HEAD_DIMS, lambda: f"unsupported head_dim {D} (allowed: 16,32,64,128)")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    return _forward(q, k, v, causal, sm_scale, return_softmax_lse, gqa=True)


# Public alias (reference: triton_fa.py:401)
flash_attn_volta = flash_attn_forward
