"""Autograd-aware FlashAttention: ``flash_attn(q, k, v, causal, sm_scale)``.

Same contract as the reference (flash_attn_volta/autograd.py:19-59): the
forward runs ``flash_attn_forward(..., return_softmax_lse=True)`` and saves
(q, k, v, out, lse); the backward makes ``do`` contiguous fp16 and calls
``flash_attn_backward``; gradients are returned for (q, k, v) and None for
(causal, sm_scale).

Host cost per step.  A call signature with a launch plan (forward.py)
runs through the C++ autograd node of ``_fa_torch`` (csrc/fa_torch.cpp):
the forward and the node are recorded in C++, and the backward runs on the
autograd engine's thread without taking the GIL, which a Python backward
node must take while the thread that called backward() waits for it.  The
Python Function below is the path for everything else (general layouts,
D = 16, functorch transforms, torch.compile tracing, or no _fa_torch
build); it keeps the forward's plan on the context and runs the backward
plan paired with it.  ``_apply`` skips torch's Python-level
``Function.apply`` wrapper when no functorch transform is active (it only
binds defaults there and unwraps dead functorch wrappers, which this does
with the same C call).
"""
from __future__ import annotations

import torch

from . import backward as _bw
from .backward import backward_planned
from .forward import _GENERIC, forward_planned, fwd_plan

try:
    from . import _fa_torch as _cpp
except ImportError:         # not built: the Python Function carries every call
    _cpp = None

_transforms_active = torch._C._are_functorch_transforms_active
_compiling = getattr(torch.compiler, "is_compiling", lambda: False)


def _saved_backward(ctx, do, gqa):
    q, k, v, out, lse = ctx.saved_tensors
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    if not do.is_contiguous():
        do = do.contiguous()
    plan = ctx.plan
    if plan is not None:
        bwd = plan.bwd if plan.bwd is not None else plan.make_bwd()
        r = bwd(do, q, k, v, out, lse)
        if r is not None:
            return r[0], r[1], r[2], None, None
    dq, dk, dv = backward_planned(do, q, k, v, out, lse, ctx.causal, ctx.sm_scale, gqa)
    return dq, dk, dv, None, None


class _FlashAttnFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal: bool, sm_scale: float | None):
        out, lse, plan = forward_planned(q, k, v, causal, sm_scale, True, False)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.plan = plan
        ctx.causal = causal
        ctx.sm_scale = sm_scale
        return out

    @staticmethod
    def backward(ctx, do):
        return _saved_backward(ctx, do, False)


class _FlashAttnGqaFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal: bool, sm_scale: float | None):
        out, lse, plan = forward_planned(q, k, v, causal, sm_scale, True, True)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.plan = plan
        ctx.causal = causal
        ctx.sm_scale = sm_scale
        return out

    @staticmethod
    def backward(ctx, do):
        return _saved_backward(ctx, do, True)


def _direct_apply(cls):
    """cls.apply without the Python wrapper of torch.autograd.Function, or
    None where this torch lacks the pieces it relies on."""
    try:
        base = torch._C._FunctionBase.__dict__["apply"].__get__(None, cls)
        active = torch._C._are_functorch_transforms_active
        unwrap = torch._C._functorch.unwrap_if_dead
    except (AttributeError, KeyError):
        return None

    def apply(q, k, v, causal, sm_scale):
        if active():
            return cls.apply(q, k, v, causal, sm_scale)
        return base(unwrap(q), unwrap(k), unwrap(v), causal, sm_scale)
    return apply


_apply = _direct_apply(_FlashAttnFn) or _FlashAttnFn.apply
_apply_gqa = _direct_apply(_FlashAttnGqaFn) or _FlashAttnGqaFn.apply


def flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               causal: bool = False, sm_scale: float | None = None) -> torch.Tensor:
    """Autograd-aware FlashAttention over (B, N, H, D) fp16 tensors.

    Args:
        q, k, v: (B, N, H, D) fp16 on the GPU. D in {16, 32, 64, 128}.
        causal: lower-triangular mask if True.
        sm_scale: softmax scale (default 1/sqrt(D)).

    Returns:
        out: (B, N, H, D) fp16, differentiable w.r.t. q, k, v.
    """
    if _cpp is not None and not _transforms_active() and not _compiling():
        out = _cpp_attn(q, k, v, causal, sm_scale, False)
        if out is not None:
            return out
    return _apply(q, k, v, causal, sm_scale)


def _cpp_attn(q, k, v, causal, sm_scale, gqa):
    """The C++ node's forward for a planned signature, else None."""
    plan = fwd_plan(q, k, v, causal, sm_scale, True, gqa)
    if plan is _GENERIC:
        return None
    return _cpp.attn(plan.cpp or plan.make_cpp(_cpp), q, k, v, _bw.split_workspace)


def flash_attn_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   causal: bool = False, sm_scale: float | None = None) -> torch.Tensor:
    """Autograd-aware grouped-query attention (no counterpart in the
    reference): q (B, Sq, H, D), k and v (B, Sk, Hk, D), fp16 or bf16, with H
    a multiple of Hk; causal masks bottom-right aligned (query i sees keys
    j <= i + Sk - Sq).  Returns (B, Sq, H, D) in the input dtype."""
    if _cpp is not None and not _transforms_active() and not _compiling():
        out = _cpp_attn(q, k, v, causal, sm_scale, True)
        if out is not None:
            return out
    return _apply_gqa(q, k, v, causal, sm_scale)
