"""Backward attention over (B, S, H, D) fp16 tensors on an MI355X.

Drop-in for the reference's ``flash_attn_backward``
(flash_attn_volta/triton_fa_bwd.py:587-700): same signature and return
value.  One ``fa_bwd`` call (include/fa_mi355x.h) runs two gfx950 kernels
on the current stream: the dQ kernel, which also computes
delta = rowsum(dO * O) (the reference's separate pre-pass) into the
caller-owned workspace, then the dK/dV kernel, which reads it.  No permute
copies; D = 16 is zero-padded to 32 like the forward.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _capi, _runtime
from ._runtime import VP
from .forward import (_DTYPES, _GENERIC, _MAX_PLANS, NATIVE_HEAD_DIMS, SUPPORTED_HEAD_DIMS,
                      _check_gqa, _contiguous_strides, _kernel_ready, _layout_ready, _on_device,
                      _pad_d, _require, _stream_ptr, _strides_c, kernel_strides)


def flash_attn_backward(
    do: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    causal: bool = False,
    sm_scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """FlashAttention backward: fp16 in/out, fp32 accumulation.

    Args:
        do: (B, N, H, D) fp16, gradient of the loss w.r.t. the output.
        q, k, v, o: (B, N, H, D) fp16 forward inputs and output.
        lse: (B, H, N) fp32 from ``flash_attn_forward(..., return_softmax_lse=True)``.
        causal, sm_scale: must match the forward call.

    Returns:
        (dq, dk, dv), each (B, N, H, D) fp16 contiguous.
    """
    return backward_planned(do, q, k, v, o, lse, causal, sm_scale, False)


def _validate_bwd(do, q, k, v, o, lse):
    _require(q.is_cuda and k.is_cuda and v.is_cuda and o.is_cuda and do.is_cuda,
             "tensors must be on CUDA")
    _require(q.dtype == torch.float16 == k.dtype == v.dtype == o.dtype == do.dtype, "fp16 only")
    _require(lse.dtype == torch.float32, "lse must be fp32")
    _require(q.shape == k.shape == v.shape == o.shape == do.shape, "shape mismatch")
    _require(q.dim() == 4, lambda: f"expected (B, N, H, D) tensors, got {tuple(q.shape)}")
    B, N, H, D = q.shape
    _require(D in SUPPORTED_HEAD_DIMS, lambda: f"unsupported head_dim {D}")
    _require(tuple(lse.shape) == (B, H, N), lambda: f"lse shape {tuple(lse.shape)} expected ({B},{H},{N})")
    _require(lse.is_cuda and lse.device == q.device, "lse must be on the same device")


def _validate_bwd_gqa(do, q, k, v, o, lse):
    _require(q.is_cuda and k.is_cuda and v.is_cuda and o.is_cuda and do.is_cuda,
             "tensors must be on CUDA")
    _require(q.dtype in _DTYPES and q.dtype == k.dtype == v.dtype == o.dtype == do.dtype,
             "fp16 or bf16 only, all alike")
    _require(lse.dtype == torch.float32, "lse must be fp32")
    _check_gqa(q, k, v)
    _require(q.shape == o.shape == do.shape, "q, o and do shapes differ")
    B, N, H, D = q.shape
    _require(D in SUPPORTED_HEAD_DIMS, lambda: f"unsupported head_dim {D}")
    _require(tuple(lse.shape) == (B, H, N), lambda: f"lse shape {tuple(lse.shape)} expected ({B},{H},{N})")
    _require(lse.is_cuda and lse.device == q.device, "lse must be on the same device")


# Launch plans by call signature (see forward.py's _FWD_PLANS).
_BWD_PLANS: dict = {}


def backward_planned(do, q, k, v, o, lse, causal, sm_scale, gqa):
    """(dq, dk, dv) through the launch plan of this call signature, built
    (after the argument checks) the first time it is seen."""
    key = (do.shape, q.shape, k.shape, v.shape, o.shape, lse.shape, do.stride(), q.stride(),
           k.stride(), v.stride(), o.stride(), lse.stride(), do.dtype, q.dtype, k.dtype, v.dtype,
           o.dtype, lse.dtype, do.device, q.device, k.device, v.device, o.device, lse.device,
           causal, sm_scale, gqa)
    try:
        plan = _BWD_PLANS.get(key)
    except TypeError:           # an unhashable causal / sm_scale: no caching
        key = plan = None
    if plan is None:
        (_validate_bwd_gqa if gqa else _validate_bwd)(do, q, k, v, o, lse)
        plan = _GENERIC
        B, N, H, D = q.shape
        if (D in NATIVE_HEAD_DIMS and q.numel() and k.numel() and lse.is_contiguous()
                and all(_layout_ready(t) for t in (do, q, k, v, o))):
            plan = _BwdPlan(B, N, k.shape[1], H, k.shape[2], D,
                            [kernel_strides(t) for t in (do, q, k, v, o)], q.stride(), k.stride(),
                            q.dtype, q.device, causal,
                            1.0 / math.sqrt(D) if sm_scale is None else sm_scale, gqa)
        if key is not None:
            if len(_BWD_PLANS) >= _MAX_PLANS:
                _BWD_PLANS.clear()
            _BWD_PLANS[key] = plan
    if plan is not _GENERIC:
        r = plan(do, q, k, v, o, lse)
        if r is not None:
            return r
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[3])
    return _backward(do, q, k, v, o, lse, causal, sm_scale, gqa)


class _BwdPlan:
    """Launch plan of one backward call signature whose tensors the kernels
    read in place: fa_bwd / fa_bwd_gqa and its size / stride / scale / flag
    arguments, converted once, with both workspace sizes (split schedule or
    delta only, by ``split_workspace`` at call time).  A call allocates dQ,
    dK, dV, takes the stream's cached workspace and passes the pointers; the
    general path (_backward) gives the same results."""
    __slots__ = ("fn", "name", "rest", "ws_split", "ws_plain", "q_shape", "k_shape", "q_like",
                 "k_like", "dtype", "device", "idx")

    def __init__(self, B, Sq, Sk, H, Hk, D, in_strides, q_stride, k_stride, dtype, device,
                 causal, sm_scale, gqa):
        lib = _capi.load()
        self.q_shape, self.k_shape = (B, Sq, H, D), (B, Sk, Hk, D)
        q_st, k_st = _contiguous_strides(self.q_shape), _contiguous_strides(self.k_shape)
        self.q_like, self.k_like = tuple(q_stride) == q_st, tuple(k_stride) == k_st
        self.dtype, self.device, self.idx = dtype, device, device.index
        sq_, sk_ = _strides_c(self.q_shape, q_st), _strides_c(self.k_shape, k_st)
        st = (*in_strides, sq_, sk_, sk_)
        c = int(bool(causal))
        # (bytes, the same as a C size_t argument)
        n = int(lib.fa_bwd_workspace_bytes(B, Sq, H, D))
        self.ws_plain = (n, ctypes.c_size_t(n))
        n = int(lib.fa_bwd_gqa_workspace_bytes(B, Sq, Sk, H, Hk, D, c))
        self.ws_split = (n, ctypes.c_size_t(n))
        if gqa:
            self.name = "fa_bwd_gqa"
            self.rest = _runtime.convert(self.name, 11, (B, Sq, Sk, H, Hk, D, *st, float(sm_scale),
                                                         c, _DTYPES[dtype]))
        else:
            self.name = "fa_bwd"
            self.rest = _runtime.convert(self.name, 11, (B, Sq, H, D, *st, float(sm_scale), c))
        self.fn = _runtime.entry(self.name)

    def __call__(self, do, q, k, v, o, lse):
        """(dq, dk, dv), or None when a data pointer is not 16-byte aligned
        (the general path copies those)."""
        ptrs = (do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr())
        if (ptrs[0] | ptrs[1] | ptrs[2] | ptrs[3] | ptrs[4]) & 15:
            return None
        dq = (torch.empty_like(q) if self.q_like
              else torch.empty(self.q_shape, dtype=self.dtype, device=self.device))
        # separate allocations: outputs of the registered custom op (ops.py)
        # must not share storage
        if self.k_like:
            dk, dv = torch.empty_like(k), torch.empty_like(k)
        else:
            dk = torch.empty(self.k_shape, dtype=self.dtype, device=self.device)
            dv = torch.empty(self.k_shape, dtype=self.dtype, device=self.device)
        if _runtime.current_device() == self.idx:
            rc = self._launch(ptrs, lse, dq, dk, dv)
        else:
            with _runtime.on_device(self.idx):
                rc = self._launch(ptrs, lse, dq, dk, dv)
        if rc:
            _capi.check(rc, self.name)
        return dq, dk, dv

    def _launch(self, ptrs, lse, dq, dk, dv):
        stream = _runtime.stream_ptr(self.idx)
        nbytes, c_nbytes = self.ws_split if split_workspace else self.ws_plain
        ws = _runtime.workspace(nbytes, self.device, stream)
        return self.fn(VP(ptrs[0]), VP(ptrs[1]), VP(ptrs[2]), VP(ptrs[3]), VP(ptrs[4]),
                       VP(lse.data_ptr()), VP(dq.data_ptr()), VP(dk.data_ptr()), VP(dv.data_ptr()),
                       VP(ws.data_ptr()), c_nbytes, *self.rest, VP(stream))


def _backward(do, q, k, v, o, lse, causal, sm_scale, gqa):
    D = q.shape[-1]
    if D not in NATIVE_HEAD_DIMS:
        dq, dk, dv = _run_bwd(_pad_d(do, 32), _pad_d(q, 32), _pad_d(k, 32), _pad_d(v, 32),
                              _pad_d(o, 32), lse, causal, sm_scale, gqa)
        return dq[..., :D].contiguous(), dk[..., :D].contiguous(), dv[..., :D].contiguous()
    return _run_bwd(do, q, k, v, o, lse, causal, sm_scale, gqa)


# The backward's workspace: with split_workspace (the default) it asks for
# fa_bwd_gqa_workspace_bytes, with which small causal D = 64 / 128 grids run
# their split schedule (longest key / query blocks swept by two workgroups;
# 8-20 % faster on those grids, at up to 80 MiB of fp32 partials); set it
# to False to cap the workspace at delta's B * H * Sq * 4 bytes (the
# unsplit schedule, same results to rounding).  The workspace is cached per
# stream and reused by later calls (_runtime.workspace;
# flash_attn_volta.release_workspaces() frees it).
split_workspace = True

_WS_BYTES = {}


def _run_bwd(do, q, k, v, o, lse, causal, sm_scale, gqa):
    lib = _capi.load()
    B, N, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    do, q, k, v, o = (_kernel_ready(t) for t in (do, q, k, v, o))
    lse = lse.contiguous()
    dq = torch.empty((B, N, H, D), dtype=q.dtype, device=q.device)
    # separate allocations: outputs of the registered custom op (ops.py)
    # must not share storage
    dk = torch.empty((B, Sk, Hk, D), dtype=q.dtype, device=q.device)
    dv = torch.empty_like(dk)
    if dq.numel() == 0 or dk.numel() == 0:
        # nothing attends to anything: every gradient is zero
        for t in (dq, dk, dv):
            t.zero_()
        return dq, dk, dv
    sq_, sk_ = kernel_strides(dq), kernel_strides(dk)
    st = (kernel_strides(do), kernel_strides(q), kernel_strides(k), kernel_strides(v),
          kernel_strides(o), sq_, sk_, sk_)
    with _on_device(q.device):
        # the size that lets small causal D = 64 / 128 grids split their
        # longest key / query blocks (fa_bwd_gqa_workspace_bytes); delta
        # alone otherwise
        key = (B, N, Sk, H, Hk, D, bool(causal), split_workspace)
        ws_bytes = _WS_BYTES.get(key)
        if ws_bytes is None:
            if split_workspace:
                ws_bytes = lib.fa_bwd_gqa_workspace_bytes(B, N, Sk, H, Hk, D, int(bool(causal)))
            else:
                ws_bytes = lib.fa_bwd_workspace_bytes(B, N, H, D)
            _WS_BYTES[key] = ws_bytes
        stream = _stream_ptr(q.device)
        ws = _runtime.workspace(ws_bytes, q.device, stream)
        if gqa:
            rc = lib.fa_bwd_gqa(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                o.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                dv.data_ptr(), ws.data_ptr(), ws_bytes, B, N, Sk, H, Hk, D, *st,
                                float(sm_scale), int(bool(causal)), _DTYPES[q.dtype], stream)
        else:
            rc = lib.fa_bwd(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                            ws.data_ptr(), ws_bytes, B, N, H, D, *st,
                            float(sm_scale), int(bool(causal)), stream)
    _capi.check(rc, "fa_bwd_gqa" if gqa else "fa_bwd")
    return dq, dk, dv


def flash_attn_backward_gqa(
    do: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    causal: bool = False,
    sm_scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of ``flash_attn_forward_gqa`` (no counterpart in the
    reference).  do, q, o: (B, Sq, H, D); k, v: (B, Sk, Hk, D); lse:
    (B, H, Sq).  Returns dq (B, Sq, H, D) and dk, dv (B, Sk, Hk, D), the
    latter summed over the query heads that share each key/value head.
    fp16 or bf16 (every tensor alike, gradients in the same dtype)."""
    return backward_planned(do, q, k, v, o, lse, causal, sm_scale, True)


def bwd_preprocess(o: torch.Tensor, do: torch.Tensor) -> torch.Tensor:
    """delta[b, h, s] = sum_d o * do in fp32, (B, H, S) -- the pre-pass of the
    backward (reference: triton_fa_bwd.py:649-650), exposed for testing."""
    lib = _capi.load()
    _require(o.shape == do.shape and o.dim() == 4, "shape mismatch")
    _require(o.dtype == torch.float16 == do.dtype, "fp16 only")
    B, N, H, D = o.shape
    _require(D in NATIVE_HEAD_DIMS, lambda: f"unsupported head_dim {D}")
    o, do = _kernel_ready(o), _kernel_ready(do)
    delta = torch.empty((B, H, N), dtype=torch.float32, device=o.device)
    with _on_device(o.device):
        rc = lib.fa_bwd_preprocess(o.data_ptr(), do.data_ptr(), delta.data_ptr(), None, B, N, H,
                                   D, kernel_strides(o), kernel_strides(do), _stream_ptr(o.device))
    _capi.check(rc, "fa_bwd_preprocess")
    return delta
