"""Autograd-aware FlashAttention: ``flash_attn(q, k, v, causal, sm_scale)``.

Same contract as the reference (flash_attn_volta/autograd.py:19-59): the
forward runs ``flash_attn_forward(..., return_softmax_lse=True)`` and saves
(q, k, v, out, lse); the backward makes ``do`` contiguous fp16 and calls
``flash_attn_backward``; gradients are returned for (q, k, v) and None for
(causal, sm_scale).
"""
from __future__ import annotations

import math

import torch

from .backward import flash_attn_backward, flash_attn_backward_gqa
from .forward import flash_attn_forward, flash_attn_forward_gqa


class _FlashAttnFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal: bool, sm_scale: float | None):
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(q.shape[-1])
        out, lse = flash_attn_forward(q, k, v, causal=causal, sm_scale=sm_scale,
                                      return_softmax_lse=True)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal = causal
        ctx.sm_scale = sm_scale
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, out, lse = ctx.saved_tensors
        do = do.contiguous()
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        dq, dk, dv = flash_attn_backward(do, q, k, v, out, lse,
                                         causal=ctx.causal, sm_scale=ctx.sm_scale)
        return dq, dk, dv, None, None


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
    return _FlashAttnFn.apply(q, k, v, causal, sm_scale)


class _FlashAttnGqaFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal: bool, sm_scale: float | None):
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(q.shape[-1])
        out, lse = flash_attn_forward_gqa(q, k, v, causal=causal, sm_scale=sm_scale,
                                          return_softmax_lse=True)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal = causal
        ctx.sm_scale = sm_scale
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, out, lse = ctx.saved_tensors
        do = do.contiguous()
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        dq, dk, dv = flash_attn_backward_gqa(do, q, k, v, out, lse,
                                             causal=ctx.causal, sm_scale=ctx.sm_scale)
        return dq, dk, dv, None, None


def flash_attn_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   causal: bool = False, sm_scale: float | None = None) -> torch.Tensor:
    """Autograd-aware grouped-query attention (no counterpart in the
    reference): q (B, Sq, H, D), k and v (B, Sk, Hk, D), fp16 or bf16, with H
    a multiple of Hk; causal masks bottom-right aligned (query i sees keys
    j <= i + Sk - Sq).  Returns (B, Sq, H, D) in the input dtype."""
    return _FlashAttnGqaFn.apply(q, k, v, causal, sm_scale)
