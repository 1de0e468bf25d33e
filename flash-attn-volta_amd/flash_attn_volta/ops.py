"""FlashAttention as ``torch.library`` custom ops, for ``torch.compile``.

The reference's boundary notes this as optional (its callers are plain
autograd code); here it is: ``flash_attn_volta::fwd`` and
``flash_attn_volta::bwd`` are registered with fake-tensor implementations
(output shapes and dtypes without running anything) and an autograd
formula, so a compiled graph keeps the attention call as one opaque node
instead of breaking the graph at a Python autograd Function.  The ops run
the same C-ABI kernels as ``flash_attn_gqa`` (grouped heads, ``Sq != Sk``,
fp16 or bf16).

    flash_attn_op(q, k, v, causal=False, sm_scale=None) -> out
"""
from __future__ import annotations

import math

import torch

from .backward import flash_attn_backward_gqa
from .forward import flash_attn_forward_gqa

__all__ = ["flash_attn_op"]


@torch.library.custom_op("flash_attn_volta::fwd", mutates_args=(), device_types="cuda")
def _fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
         sm_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    out, lse = flash_attn_forward_gqa(q, k, v, causal=causal, sm_scale=sm_scale,
                                      return_softmax_lse=True)
    return out, lse


@_fwd.register_fake
def _fwd_fake(q, k, v, causal, sm_scale):
    B, Sq, H, D = q.shape
    out = q.new_empty((B, Sq, H, D))
    lse = q.new_empty((B, H, Sq), dtype=torch.float32)
    return out, lse


@torch.library.custom_op("flash_attn_volta::bwd", mutates_args=(), device_types="cuda")
def _bwd(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
         lse: torch.Tensor, causal: bool,
         sm_scale: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return flash_attn_backward_gqa(do, q, k, v, o, lse, causal=causal, sm_scale=sm_scale)


@_bwd.register_fake
def _bwd_fake(do, q, k, v, o, lse, causal, sm_scale):
    return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape)


def _setup_context(ctx, inputs, output):
    q, k, v, causal, sm_scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse)
    ctx.causal = causal
    ctx.sm_scale = sm_scale
    ctx.mark_non_differentiable(lse)


def _backward(ctx, dout, _dlse):
    q, k, v, out, lse = ctx.saved_tensors
    dout = dout.contiguous()
    if dout.dtype != q.dtype:
        dout = dout.to(q.dtype)
    dq, dk, dv = torch.ops.flash_attn_volta.bwd(dout, q, k, v, out, lse, ctx.causal,
                                                ctx.sm_scale)
    return dq, dk, dv, None, None


_fwd.register_autograd(_backward, setup_context=_setup_context)


def flash_attn_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                  sm_scale: float | None = None) -> torch.Tensor:
    """``flash_attn_gqa`` through the registered custom ops (differentiable,
    traceable by ``torch.compile``).  q (B, Sq, H, D); k, v (B, Sk, Hk, D)
    with H a multiple of Hk; fp16 or bf16; returns (B, Sq, H, D)."""
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    out, _ = torch.ops.flash_attn_volta.fwd(q, k, v, bool(causal), float(sm_scale))
    return out
