"""CPU oracle for the fused QK-norm + rotary prologue -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py`` may import this
module, and only as the checker.  The product path (flash_attn_volta.rope)
never touches it.

What it restates, in float64, from the mathematics: the prologue the
reference's HF patch runs before its attention call, which the reference
leaves to the third-party transformers library --

* Qwen3 (patch_hf.py:291-303): ``q = q_norm(q)``, ``k = k_norm(k)`` with
  transformers' Qwen3RMSNorm (per head over the last dimension:
  ``w * x / sqrt(mean(x^2) + eps)``), then ``apply_rotary_pos_emb``;
* Qwen2 / Llama (patch_hf.py:177, :462): ``apply_rotary_pos_emb`` alone.

``apply_rotary_pos_emb(q, k, cos, sin)`` is ``q * cos + rotate_half(q) * sin``
with ``rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])`` (transformers;
the reference targets 4.44 and the installed 5.15 has the same definition),
cos/sin of shape (B, S, D) broadcast over heads.  The reference's tensors
are (B, H, S, D); here, as in the kernels, (B, S, H, D).

Functions:
  rope_qk_fwd  -- forward of both sides (norm optional per side).
  rope_qk_bwd  -- the analytic backward: dq, dk, and the norm weights'
                  gradients (sum over rows of dy * n).
  rope_tables  -- cos/sin exactly as transformers' default rotary embedding
                  builds them (inv_freq = base^(-2i/D) in fp32, angle =
                  position * inv_freq in fp32, emb = cat(freqs, freqs),
                  cos/sin cast to the model dtype).
  make_rope_inputs -- seeded fp16/bf16 inputs for tests and the bench.

How each function is pinned (tests/test_oracle_rope.py):
  rope_qk_fwd : golden vectors written by transformers' own
                apply_rotary_pos_emb and Qwen3RMSNorm in float64
                (tests/golden/make_rope_golden.py); closed forms (position
                0 is the identity, each rotation pair keeps its norm, the
                rotation by -theta undoes it, unit-weight RMSNorm output has
                mean square 1 when eps = 0).
  rope_qk_bwd : golden vectors from torch float64 autograd through the same
                transformers functions; central finite differences of
                rope_qk_fwd; the adjoint identity <R x, g> = <x, R^T g>.
  Planted mistakes (interleaved-pair rotation, the opposite rotation sign,
  a norm without the weight) fail these checks.
"""
from __future__ import annotations

import numpy as np

__all__ = ["rope_qk_fwd", "rope_qk_bwd", "rope_tables", "make_rope_inputs"]


def _f64(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def _table(c, B, S, D):
    """cos/sin as (B, S, 1, D) for broadcasting over heads."""
    c = _f64(c)
    if c.ndim == 2:
        c = c[None]
    assert c.shape[-2:] == (S, D) and c.shape[0] in (1, B), c.shape
    return c[:, :, None, :]


def _rotate_half(x):
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def _unrotate_half(g):
    """Adjoint of _rotate_half: <rotate_half(x), g> = <x, _unrotate_half(g)>."""
    h = g.shape[-1] // 2
    return np.concatenate([g[..., h:], -g[..., :h]], axis=-1)


def _norm(x, w, eps):
    """(n, r) with n = x * r, r = 1 / sqrt(mean(x^2) + eps) per row."""
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r, r


def _side_fwd(x, c, s, w, eps):
    y = x
    if w is not None:
        n, _ = _norm(x, w, eps)
        y = n * w
    return y * c + _rotate_half(y) * s


def rope_qk_fwd(q, k, cos, sin, q_norm_weight=None, k_norm_weight=None, eps=1e-6):
    """float64 (q_out, k_out) of the fused prologue; q (B,S,H,D), k (B,S,Hk,D)."""
    q, k = _f64(q), _f64(k)
    B, S, _, D = q.shape
    c, s = _table(cos, B, S, D), _table(sin, B, S, D)
    return (_side_fwd(q, c, s, _f64(q_norm_weight), eps),
            _side_fwd(k, c, s, _f64(k_norm_weight), eps))


def _side_bwd(g, x, c, s, w, eps):
    # out = y * c + rotate_half(y) * s  =>  dy = g * c + rotate_half^T(g * s)
    dy = g * c + _unrotate_half(g * s)
    if w is None:
        return dy, None
    n, r = _norm(x, w, eps)
    dw = np.sum(dy * n, axis=tuple(range(dy.ndim - 1)))
    dn = dy * w
    dx = r * (dn - n * np.mean(dn * n, axis=-1, keepdims=True))
    return dx, dw


def rope_qk_bwd(dq_out, dk_out, q, k, cos, sin, q_norm_weight=None, k_norm_weight=None,
                eps=1e-6):
    """float64 (dq, dk, dq_norm_weight, dk_norm_weight); a weight's gradient
    is None when that side has no norm."""
    g_q, g_k, q, k = _f64(dq_out), _f64(dk_out), _f64(q), _f64(k)
    B, S, _, D = g_q.shape
    c, s = _table(cos, B, S, D), _table(sin, B, S, D)
    dq, dwq = _side_bwd(g_q, q, c, s, _f64(q_norm_weight), eps)
    dk, dwk = _side_bwd(g_k, k, c, s, _f64(k_norm_weight), eps)
    return dq, dk, dwq, dwk


def rope_tables(positions, D, base=10000.0, dtype=None):
    """cos, sin of shape positions.shape + (D,), built the way transformers'
    default rotary embedding does (fp32 angles, emb = cat(freqs, freqs)),
    then cast to ``dtype`` (a torch dtype) when given."""
    import torch
    pos = torch.as_tensor(positions)
    inv = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    freqs = pos.float()[..., None] * inv
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    if dtype is not None:
        cos, sin = cos.to(dtype), sin.to(dtype)
    return cos, sin


def make_rope_inputs(B, S, H, Hk, D, seed=0, dtype=None, norm=False, shared_table=False,
                     start=0):
    """Seeded CPU inputs: q (B,S,H,D), k (B,S,Hk,D), cos/sin ((1 or B), S, D),
    norm weights (D,) or None, and output gradients, all in ``dtype``
    (torch.float16 by default).  Batch b sits at positions start + b + s so
    the per-batch tables differ unless ``shared_table``."""
    import torch
    dtype = dtype or torch.float16
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, S, H, D, generator=g).to(dtype)
    k = torch.randn(B, S, Hk, D, generator=g).to(dtype)
    dq = torch.randn(B, S, H, D, generator=g).to(dtype)
    dk = torch.randn(B, S, Hk, D, generator=g).to(dtype)
    nb = 1 if shared_table else B
    pos = start + torch.arange(S)[None, :] + torch.arange(nb)[:, None]
    cos, sin = rope_tables(pos, D, dtype=dtype)
    wq = wk = None
    if norm:
        wq = (1.0 + 0.25 * torch.randn(D, generator=g)).to(dtype)
        wk = (1.0 + 0.25 * torch.randn(D, generator=g)).to(dtype)
    return q, k, cos, sin, wq, wk, dq, dk
