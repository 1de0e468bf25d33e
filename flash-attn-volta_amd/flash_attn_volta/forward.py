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


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise FlashAttnArgumentError(msg)


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` if the kernel can read it in place (unit D stride,
    16-byte aligned base, other strides multiples of 8 elements), else a
    contiguous copy."""
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


def _stream_ptr(device: torch.device) -> int:
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
    _require(q.shape == k.shape == v.shape, f"qkv shape mismatch {q.shape} {k.shape} {v.shape}")
    _require(q.dim() == 4, f"expected (B, N, H, D) tensors, got {tuple(q.shape)}")
    _require(q.device == k.device == v.device, "q, k, v must be on one device")
    B, N, H, D = q.shape
    _require(D in SUPPORTED_HEAD_DIMS, f"unsupported head_dim {D} (allowed: 16,32,64,128)")

    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)

    if D not in NATIVE_HEAD_DIMS:
        out, lse = _run_fwd(_pad_d(q, 32), _pad_d(k, 32), _pad_d(v, 32), causal, sm_scale,
                            return_softmax_lse)
        out = out[..., :D].contiguous()
    else:
        out, lse = _run_fwd(q, k, v, causal, sm_scale, return_softmax_lse)
    if return_softmax_lse:
        return out, lse
    return out


def _run_fwd(q, k, v, causal, sm_scale, write_lse):
    lib = _capi.load()
    B, N, H, D = q.shape
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    out = torch.empty((B, N, H, D), dtype=torch.float16, device=q.device)
    lse = torch.empty((B, H, N), dtype=torch.float32, device=q.device) if write_lse else None
    if out.numel() == 0:
        if lse is not None:
            lse.fill_(float("inf"))
        return out, lse
    with _on_device(q.device):
        rc = lib.fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                        lse.data_ptr() if lse is not None else None,
                        B, N, H, D,
                        kernel_strides(q), kernel_strides(k), kernel_strides(v), kernel_strides(out),
                        float(sm_scale), int(bool(causal)), _stream_ptr(q.device))
    _capi.check(rc, "fa_fwd")
    return out, lse


# Public alias (reference: triton_fa.py:401)
flash_attn_volta = flash_attn_forward
