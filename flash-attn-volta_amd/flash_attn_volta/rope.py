"""Fused QK-norm + rotary position embedding for q and k on an MI355X.

The prologue of a Llama / Qwen2 / Qwen3 attention layer, which the
reference leaves to transformers before its kernel call (Qwen3's q_norm /
k_norm then ``apply_rotary_pos_emb``, flash_attn_volta/patch_hf.py:291-303;
``apply_rotary_pos_emb`` alone at patch_hf.py:177, :462), as one HBM pass
per direction: ``fa_rope_qk_fwd`` reads q and k once and writes the rotated
(and, for Qwen3, normalised) q and k in the (B, S, H, D) layout the
attention kernels read; ``fa_rope_qk_bwd`` maps their gradients back and
reduces the norm weights' gradients without atomics.  In eager transformers
the same prologue is about ten elementwise kernels per tensor and
direction.

    q_out, k_out = apply_rotary_qk(q, k, cos, sin)                      # Llama, Qwen2
    q_out, k_out = apply_rotary_qk(q, k, cos, sin, q_norm.weight,
                                   k_norm.weight, eps)                  # Qwen3

Semantics per row x of D elements (one (b, s, head)):
    y = w * x / sqrt(mean(x^2) + eps)    (with a norm weight w; else y = x)
    out = y * cos + rotate_half(y) * sin,   rotate_half(y) = cat(-y[D/2:], y[:D/2])
computed in fp32 and rounded once (transformers rounds after the norm, the
weight product and each term of the rotation).
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi
from .forward import (FlashAttnArgumentError, _DTYPES, _kernel_ready, _on_device, _require,
                      _stream_ptr, kernel_strides)

ROPE_HEAD_DIMS = (16, 32, 64, 128)

__all__ = ["apply_rotary_qk", "rope_qk_forward", "rope_qk_backward", "ROPE_HEAD_DIMS"]


def _table(t: torch.Tensor, name: str, B: int, S: int, D: int, dtype, device) -> torch.Tensor:
    """cos / sin as a (1 or B, S, D) tensor the kernel can read: unit D
    stride, 16-byte aligned, other strides multiples of 8 elements."""
    _require(isinstance(t, torch.Tensor), lambda: f"{name} must be a tensor")
    if t.dim() == 2:
        t = t.unsqueeze(0)
    _require(t.dim() == 3 and t.shape[1:] == (S, D) and t.shape[0] in (1, B),
             f"{name} must be (B or 1, S, D) = (.., {S}, {D}), got {tuple(t.shape)}")
    _require(t.device == device, lambda: f"{name} must be on {device}")
    if t.dtype != dtype:
        t = t.to(dtype)
    ok = t.stride(2) == 1 and t.data_ptr() % 16 == 0 and \
        (t.size(1) == 1 or t.stride(1) % 8 == 0) and (t.size(0) == 1 or t.stride(0) % 8 == 0)
    return t if ok else t.contiguous()


def _table_strides(t: torch.Tensor):
    return (ctypes.c_int64 * 2)(0 if t.size(0) == 1 else int(t.stride(0)),
                                0 if t.size(1) == 1 else int(t.stride(1)))


def _weight(w, name: str, D: int, dtype, device):
    if w is None:
        return None
    _require(isinstance(w, torch.Tensor) and w.shape == (D,),
             f"{name} must be a ({D},) tensor, got {getattr(w, 'shape', type(w))}")
    _require(w.device == device, lambda: f"{name} must be on {device}")
    w = w.detach()
    if w.dtype != dtype:
        w = w.to(dtype)
    return w if w.is_contiguous() and w.data_ptr() % 16 == 0 else w.contiguous()


def _check_qk(q: torch.Tensor, k: torch.Tensor) -> None:
    _require(q.is_cuda and k.is_cuda, "q and k must be on the GPU")
    _require(q.device == k.device, "q and k must be on one device")
    _require(q.dtype in _DTYPES and q.dtype == k.dtype,
             f"fp16 or bf16 only, q and k alike (got {q.dtype}, {k.dtype})")
    _require(q.dim() == 4 and k.dim() == 4,
             f"expected (B, S, H, D) tensors, got {tuple(q.shape)} {tuple(k.shape)}")
    _require(q.shape[0] == k.shape[0] and q.shape[1] == k.shape[1] and q.shape[3] == k.shape[3],
             f"q {tuple(q.shape)} and k {tuple(k.shape)} differ outside the head dimension")
    _require(q.shape[3] in ROPE_HEAD_DIMS,
             f"unsupported head_dim {q.shape[3]} (allowed: {ROPE_HEAD_DIMS})")


def rope_qk_forward(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    q_norm_weight: torch.Tensor | None = None,
                    k_norm_weight: torch.Tensor | None = None, eps: float = 1e-6):
    """(q_out, k_out): q (B, S, H, D), k (B, S, Hk, D) fp16 or bf16 on the
    GPU (any strides with a unit D stride); cos, sin (B or 1, S, D) or
    (S, D), cast to q's dtype if needed; norm weights (D,) or None.
    Outputs are contiguous (B, S, H, D) / (B, S, Hk, D) in q's dtype."""
    _check_qk(q, k)
    B, S, H, D = q.shape
    Hk = k.shape[2]
    cos = _table(cos, "cos", B, S, D, q.dtype, q.device)
    sin = _table(sin, "sin", B, S, D, q.dtype, q.device)
    _require(cos.shape[0] == sin.shape[0], "cos and sin must have the same shape")
    wq = _weight(q_norm_weight, "q_norm_weight", D, q.dtype, q.device)
    wk = _weight(k_norm_weight, "k_norm_weight", D, q.dtype, q.device)
    q_out = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device)
    k_out = torch.empty((B, S, Hk, D), dtype=q.dtype, device=q.device)
    if q_out.numel() == 0 and k_out.numel() == 0:
        return q_out, k_out
    _require(H > 0 and Hk > 0, lambda: f"head counts must be positive, got {H}, {Hk}")
    q, k = _kernel_ready(q), _kernel_ready(k)
    lib = _capi.load()
    with _on_device(q.device):
        rc = lib.fa_rope_qk_fwd(
            q.data_ptr(), k.data_ptr(), q_out.data_ptr(), k_out.data_ptr(),
            cos.data_ptr(), sin.data_ptr(),
            wq.data_ptr() if wq is not None else None, wk.data_ptr() if wk is not None else None,
            float(eps), B, S, H, Hk, D,
            kernel_strides(q), kernel_strides(k), kernel_strides(q_out), kernel_strides(k_out),
            _table_strides(cos), _DTYPES[q.dtype], _stream_ptr(q.device))
    _capi.check(rc, "fa_rope_qk_fwd")
    return q_out, k_out


_WS_BYTES = {}


def rope_qk_backward(dq_out: torch.Tensor, dk_out: torch.Tensor, q: torch.Tensor,
                     k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     q_norm_weight: torch.Tensor | None = None,
                     k_norm_weight: torch.Tensor | None = None, eps: float = 1e-6):
    """(dq, dk, dq_norm_weight, dk_norm_weight) from the gradients of
    rope_qk_forward's outputs.  dq, dk are contiguous in q's dtype; a norm
    weight's gradient is fp32 (D,), or None for a side without a norm.  q
    and k (the forward's inputs) are read only for a normed side."""
    _check_qk(q, k)
    B, S, H, D = q.shape
    Hk = k.shape[2]
    _require(dq_out.shape == q.shape and dk_out.shape == k.shape,
             f"gradient shapes {tuple(dq_out.shape)} {tuple(dk_out.shape)} do not match "
             f"q {tuple(q.shape)} / k {tuple(k.shape)}")
    _require(dq_out.device == q.device and dk_out.device == q.device, "gradients on another device")
    if dq_out.dtype != q.dtype:
        dq_out = dq_out.to(q.dtype)
    if dk_out.dtype != q.dtype:
        dk_out = dk_out.to(q.dtype)
    cos = _table(cos, "cos", B, S, D, q.dtype, q.device)
    sin = _table(sin, "sin", B, S, D, q.dtype, q.device)
    wq = _weight(q_norm_weight, "q_norm_weight", D, q.dtype, q.device)
    wk = _weight(k_norm_weight, "k_norm_weight", D, q.dtype, q.device)
    dq = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device)
    dk = torch.empty((B, S, Hk, D), dtype=q.dtype, device=q.device)
    dwq = torch.empty(D, dtype=torch.float32, device=q.device) if wq is not None else None
    dwk = torch.empty(D, dtype=torch.float32, device=q.device) if wk is not None else None
    if dq.numel() == 0 and dk.numel() == 0:
        for dw in (dwq, dwk):
            if dw is not None:
                dw.zero_()
        return dq, dk, dwq, dwk
    lib = _capi.load()
    ws = None
    if wq is not None or wk is not None:
        key = (B, S, H, Hk, D)
        nbytes = _WS_BYTES.get(key)
        if nbytes is None:
            nbytes = _WS_BYTES[key] = int(lib.fa_rope_qk_workspace_bytes(B, S, H, Hk, D))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    dq_out, dk_out = _kernel_ready(dq_out), _kernel_ready(dk_out)
    qs, ks = _kernel_ready(q), _kernel_ready(k)
    with _on_device(q.device):
        rc = lib.fa_rope_qk_bwd(
            dq_out.data_ptr(), dk_out.data_ptr(), qs.data_ptr(), ks.data_ptr(),
            cos.data_ptr(), sin.data_ptr(),
            wq.data_ptr() if wq is not None else None, wk.data_ptr() if wk is not None else None,
            float(eps), dq.data_ptr(), dk.data_ptr(),
            dwq.data_ptr() if dwq is not None else None, dwk.data_ptr() if dwk is not None else None,
            ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
            B, S, H, Hk, D,
            kernel_strides(dq_out), kernel_strides(dk_out), kernel_strides(qs), kernel_strides(ks),
            kernel_strides(dq), kernel_strides(dk), _table_strides(cos),
            _DTYPES[q.dtype], _stream_ptr(q.device))
    _capi.check(rc, "fa_rope_qk_bwd")
    return dq, dk, dwq, dwk


class _RopeQkFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin, q_norm_weight, k_norm_weight, eps: float):
        if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
            raise FlashAttnArgumentError("apply_rotary_qk has no gradient for the cos / sin "
                                         "tables; pass them detached")
        q_out, k_out = rope_qk_forward(q, k, cos, sin, q_norm_weight, k_norm_weight, eps)
        # the forward's inputs are needed again only to recompute a norm
        ctx.save_for_backward(q if q_norm_weight is not None else None,
                              k if k_norm_weight is not None else None,
                              cos, sin, q_norm_weight, k_norm_weight)
        ctx.shapes = (q.shape, k.shape, q.dtype, q.device)
        ctx.eps = eps
        return q_out, k_out

    @staticmethod
    def backward(ctx, g_q, g_k):
        q, k, cos, sin, wq, wk = ctx.saved_tensors
        q_shape, k_shape, dtype, device = ctx.shapes
        if g_q is None:
            g_q = torch.zeros(q_shape, dtype=dtype, device=device)
        if g_k is None:
            g_k = torch.zeros(k_shape, dtype=dtype, device=device)
        # stand-ins carry shape / dtype for a side whose input was not kept
        q = q if q is not None else g_q
        k = k if k is not None else g_k
        dq, dk, dwq, dwk = rope_qk_backward(g_q, g_k, q, k, cos, sin, wq, wk, ctx.eps)
        if dwq is not None:
            dwq = dwq.to(wq.dtype)
        if dwk is not None:
            dwk = dwk.to(wk.dtype)
        return dq, dk, None, None, dwq, dwk, None


def apply_rotary_qk(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    q_norm_weight: torch.Tensor | None = None,
                    k_norm_weight: torch.Tensor | None = None, eps: float = 1e-6):
    """Autograd-aware fused prologue (no kernel counterpart in the reference,
    which calls transformers' Qwen3RMSNorm and apply_rotary_pos_emb,
    patch_hf.py:291-303).

    Args:
        q: (B, S, H, D), k: (B, S, Hk, D), fp16 or bf16 on the GPU, in the
            (B, S, heads, D) layout the projections produce (transformers'
            ``q_proj(x).view(B, S, -1, D)``), any strides with unit D stride.
        cos, sin: (B or 1, S, D) or (S, D) rotary tables, as transformers'
            rotary embedding returns them (no gradient flows to them).
        q_norm_weight, k_norm_weight: (D,) RMSNorm weights (Qwen3's q_norm /
            k_norm), or None for no norm on that side.
        eps: the norms' epsilon.

    Returns:
        (q_out, k_out): contiguous (B, S, H, D) / (B, S, Hk, D) in q's dtype,
        ready for flash_attn / flash_attn_gqa.
    """
    return _RopeQkFn.apply(q, k, cos, sin, q_norm_weight, k_norm_weight, float(eps))
