"""CPU oracle for the FlashAttention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for
``attention_ref_fp32``, as the timed CPU baseline).  The product path in
``flash_attn_volta`` never touches it.

It restates, from the mathematics, what the reference computes:

* ``attention_fwd``  -- O = softmax(sm_scale * Q K^T [+ causal -inf]) V and
  the natural-log row LSE in float64.  Follows the reference eager path
  flash_attn_volta/ref.py:9-36 (layout (B,N,H,D), causal mask = strict upper
  triangle -inf, ref.py:26-31) and the forward kernel's output contract
  triton_fa.py:146-159 (O = acc / l, LSE = m + ln l, +inf when a row sees no
  key).
* ``attention_bwd``  -- dQ, dK, dV (and delta) in float64 by the closed-form
  softmax backward the reference kernels implement: delta = rowsum(dO * O)
  from the *stored* fp16 O (triton_fa_bwd.py:649-650), P = exp(S - LSE)
  (:165), dP = dO V^T (:168-169), dS = P (dP - delta) (:172),
  dQ = sm_scale dS K (:175-178), dV = P^T dO (:415),
  dK = sm_scale dS^T Q (:426-429).
* ``attention_ref_fp32`` -- the reference's float32 eager CPU path
  (ref.py:9-36) restated in torch; this is the CPU baseline bench.py times.
* ``make_inputs`` -- the seeded fp16 inputs every test and bench uses.
* ``attention_fwd_gqa`` / ``attention_bwd_gqa`` / ``make_inputs_gqa`` --
  the same mathematics for grouped-query attention with separate query and
  key lengths (q (B,Sq,H,D), k and v (B,Sk,Hk,D), query head h reading
  key/value head h // (H // Hk), the head order of the repeat_kv the
  reference's HF patch applies, patch_hf.py:186-188), causal mask aligned
  bottom-right (query i sees keys j <= i + Sk - Sq).  The reference kernels
  have no such mode (triton_fa.py:315 asserts equal shapes).

How each function is pinned (tests/test_oracle.py):
  attention_fwd : golden vectors written by torch's float64
                  scaled_dot_product_attention (tests/golden/), the plain-C
                  brute force oracle/attention_ref.c, closed forms (S = 1,
                  causal row 0, identical keys, convex hull of V, LSE bounds,
                  LSE = logsumexp by definition).
  attention_bwd : golden vectors from torch float64 autograd, the C brute
                  force, and central finite differences of attention_fwd.
  attention_ref_fp32 : agreement with attention_fwd to fp32 rounding.
  attention_fwd_gqa / attention_bwd_gqa : golden vectors from torch's
                  float64 SDPA (enable_gqa, explicit bottom-right mask) and
                  autograd; reduction identities to the pinned square
                  functions (GQA == attention over repeat_kv-expanded K/V
                  with dK/dV summed over each group; Sq < Sk == the last Sq
                  rows of a square causal problem; Sq > Sk == empty rows
                  then a square causal problem); planted head-mapping and
                  mask-alignment mistakes that these checks catch.
"""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

__all__ = ["make_inputs", "attention_fwd", "attention_bwd", "attention_ref_fp32",
           "make_inputs_gqa", "attention_fwd_gqa", "attention_bwd_gqa"]


def make_inputs(B: int, S: int, H: int, D: int, seed: int = 0, scale: float = 1.0,
                with_grad: bool = True):
    """Seeded (B, S, H, D) fp16 inputs as torch CPU tensors.

    q, k, v come from ``torch.Generator('cpu').manual_seed(seed)`` (randn in
    fp32, cast to fp16, then multiplied by ``scale`` in fp16); dO comes from
    seed + 1.  Identical bits on every machine, so the GPU and the oracle see
    the same inputs (the reference tests seed q,k,v with 0 and the upstream
    gradient with 1: tests/test_backward.py:193-204).
    """
    import torch
    gen = torch.Generator("cpu").manual_seed(seed)
    shape = (B, S, H, D)
    q = torch.randn(shape, generator=gen, dtype=torch.float32).half()
    k = torch.randn(shape, generator=gen, dtype=torch.float32).half()
    v = torch.randn(shape, generator=gen, dtype=torch.float32).half()
    if scale != 1.0:
        q, k, v = q * scale, k * scale, v * scale
    if not with_grad:
        return q, k, v
    gen2 = torch.Generator("cpu").manual_seed(seed + 1)
    do = torch.randn(shape, generator=gen2, dtype=torch.float32).half()
    if scale != 1.0:
        do = do * scale
    return q, k, v, do


def make_inputs_gqa(B: int, Sq: int, Sk: int, H: int, Hk: int, D: int, seed: int = 0,
                    scale: float = 1.0, dtype=None):
    """Seeded 16-bit inputs for the grouped-query functions: q (B,Sq,H,D),
    k and v (B,Sk,Hk,D) from ``Generator('cpu').manual_seed(seed)`` (randn
    fp32 -> ``dtype``, fp16 by default, times ``scale``), dO (B,Sq,H,D) from
    seed + 1."""
    import torch
    dtype = torch.float16 if dtype is None else dtype
    gen = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn((B, Sq, H, D), generator=gen, dtype=torch.float32).to(dtype)
    k = torch.randn((B, Sk, Hk, D), generator=gen, dtype=torch.float32).to(dtype)
    v = torch.randn((B, Sk, Hk, D), generator=gen, dtype=torch.float32).to(dtype)
    gen2 = torch.Generator("cpu").manual_seed(seed + 1)
    do = torch.randn((B, Sq, H, D), generator=gen2, dtype=torch.float32).to(dtype)
    if scale != 1.0:
        q, k, v, do = q * scale, k * scale, v * scale, do * scale
    return q, k, v, do


def _np64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


_UPPER = {}


def _upper(n: int, nk: int | None = None, off: int = 0) -> np.ndarray:
    """Boolean mask of the causally hidden scores (j > i + off) of an
    n x nk score matrix; n x n with off = 0 is the strict upper triangle."""
    nk = n if nk is None else nk
    key = (n, nk, off)
    m = _UPPER.get(key)
    if m is None:
        m = np.triu(np.ones((n, nk), dtype=bool), k=1 + off)
        _UPPER.clear()
        _UPPER[key] = m
    return m


def _scores(qh, kh, sm_scale, causal, off: int = 0):
    """sm_scale * q k^T for one (b, h), with the causally hidden scores
    (key j > query i + off; off = 0 is ref.py:25-31's strict upper
    triangle) set to -inf."""
    s = qh @ kh.T
    s *= sm_scale
    if causal:
        np.putmask(s, _upper(s.shape[0], s.shape[1], off), -np.inf)
    return s


def _fwd_head(qh, kh, vh, sm_scale, causal, off: int = 0):
    s = _scores(qh, kh, sm_scale, causal, off)
    m = s.max(axis=1, keepdims=True)
    empty = ~np.isfinite(m[:, 0])
    m_safe = np.where(np.isfinite(m), m, 0.0)
    s -= m_safe
    e = np.exp(s, out=s)
    l = e.sum(axis=1, keepdims=True)
    e /= np.where(l > 0, l, 1.0)
    o = e @ vh
    lse = np.where(empty, np.inf, m_safe[:, 0] + np.log(np.where(l[:, 0] > 0, l[:, 0], 1.0)))
    return o, lse


def _workers() -> int:
    return max(1, min(8, os.cpu_count() or 1))


def _map_heads(fn, B, H):
    """Run fn(b, h) for every (b, h); heads are independent, so a thread pool
    (numpy releases the GIL inside BLAS and ufuncs) only changes speed."""
    pairs = [(b, h) for b in range(B) for h in range(H)]
    if len(pairs) == 1:
        return [fn(*pairs[0])]
    with ThreadPoolExecutor(_workers()) as ex:
        return list(ex.map(lambda bh: fn(*bh), pairs))


def attention_fwd(q, k, v, causal: bool = False, sm_scale: float | None = None):
    """float64 attention. Returns (o (B,S,H,D), lse (B,H,S)), natural log."""
    q, k, v = _np64(q), _np64(k), _np64(v)
    B, S, H, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    o = np.zeros((B, S, H, D))
    lse = np.zeros((B, H, S))
    res = _map_heads(lambda b, h: _fwd_head(q[b, :, h], k[b, :, h], v[b, :, h], sm_scale, causal),
                     B, H)
    for (b, h), (oh, lh) in zip([(b, h) for b in range(B) for h in range(H)], res):
        o[b, :, h] = oh
        lse[b, h] = lh
    return o, lse


def _bwd_head(qh, kh, vh, doh, oh, sm_scale, causal, off: int = 0):
    s = _scores(qh, kh, sm_scale, causal, off)
    m = s.max(axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    s -= m
    p = np.exp(s, out=s)
    l = p.sum(axis=1, keepdims=True)
    p /= np.where(l > 0, l, 1.0)
    dl = (oh * doh).sum(axis=1)
    dv = p.T @ doh
    ds = doh @ vh.T
    ds -= dl[:, None]
    ds *= p
    dq = sm_scale * (ds @ kh)
    dk = sm_scale * (ds.T @ qh)
    return dq, dk, dv, dl


def attention_bwd(do, q, k, v, causal: bool = False, sm_scale: float | None = None, o=None):
    """float64 gradients of L = <O, dO>. Returns (dq, dk, dv, delta).

    ``o`` is the forward output the backward is given (the fp16-stored O in
    the reference, triton_fa_bwd.py:649-650); if None the exact float64 O is
    used, which makes delta exactly rowsum(dO * O).
    """
    do, q, k, v = _np64(do), _np64(q), _np64(k), _np64(v)
    B, S, H, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if o is None:
        o, _ = attention_fwd(q, k, v, causal, sm_scale)
    o = _np64(o)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    delta = np.zeros((B, H, S))
    res = _map_heads(lambda b, h: _bwd_head(q[b, :, h], k[b, :, h], v[b, :, h], do[b, :, h],
                                            o[b, :, h], sm_scale, causal), B, H)
    for (b, h), (gq, gk, gv, dl) in zip([(b, h) for b in range(B) for h in range(H)], res):
        dq[b, :, h], dk[b, :, h], dv[b, :, h], delta[b, h] = gq, gk, gv, dl
    return dq, dk, dv, delta


def attention_fwd_gqa(q, k, v, causal: bool = False, sm_scale: float | None = None):
    """float64 grouped-query attention: q (B,Sq,H,D), k and v (B,Sk,Hk,D).
    Query head h reads key/value head h // (H // Hk); causal hides key j
    from query i when j > i + Sk - Sq.  Returns (o (B,Sq,H,D),
    lse (B,H,Sq)); a row with no visible key has o = 0, lse = +inf."""
    q, k, v = _np64(q), _np64(k), _np64(v)
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    grp = H // Hk
    off = Sk - Sq
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    o = np.zeros((B, Sq, H, D))
    lse = np.zeros((B, H, Sq))
    res = _map_heads(lambda b, h: _fwd_head(q[b, :, h], k[b, :, h // grp], v[b, :, h // grp],
                                            sm_scale, causal, off), B, H)
    for (b, h), (oh, lh) in zip([(b, h) for b in range(B) for h in range(H)], res):
        o[b, :, h] = oh
        lse[b, h] = lh
    return o, lse


def attention_bwd_gqa(do, q, k, v, causal: bool = False, sm_scale: float | None = None, o=None):
    """float64 gradients of attention_fwd_gqa's L = <O, dO>.  Returns
    (dq (B,Sq,H,D), dk, dv (B,Sk,Hk,D) summed over each key/value head's
    query heads, delta (B,H,Sq)); ``o`` as in attention_bwd."""
    do, q, k, v = _np64(do), _np64(q), _np64(k), _np64(v)
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    grp = H // Hk
    off = Sk - Sq
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if o is None:
        o, _ = attention_fwd_gqa(q, k, v, causal, sm_scale)
    o = _np64(o)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    delta = np.zeros((B, H, Sq))
    res = _map_heads(lambda b, h: _bwd_head(q[b, :, h], k[b, :, h // grp], v[b, :, h // grp],
                                            do[b, :, h], o[b, :, h], sm_scale, causal, off), B, H)
    for (b, h), (gq, gk, gv, dl) in zip([(b, h) for b in range(B) for h in range(H)], res):
        dq[b, :, h] = gq
        dk[b, :, h // grp] += gk
        dv[b, :, h // grp] += gv
        delta[b, h] = dl
    return dq, dk, dv, delta


def attention_ref_fp32(q, k, v, causal: bool = False, sm_scale: float | None = None):
    """The reference's float32 eager CPU path (ref.py:9-36), restated in torch:
    permute to (B,H,N,D), fp32 scores, -inf strict upper triangle when causal,
    softmax, PV, permute back, cast to fp16.  Differentiable (autograd runs
    through it for the fwd+bwd CPU baseline)."""
    import torch
    B, N, H, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    q_ = q.permute(0, 2, 1, 3).float()
    k_ = k.permute(0, 2, 1, 3).float()
    v_ = v.permute(0, 2, 1, 3).float()
    scores = torch.matmul(q_, k_.transpose(-2, -1)) * sm_scale
    if causal:
        mask = torch.triu(torch.full((N, N), float("-inf"), dtype=torch.float32), diagonal=1)
        scores = scores + mask
    probs = torch.softmax(scores, dim=-1)
    out = torch.matmul(probs, v_)
    return out.permute(0, 2, 1, 3).contiguous().to(torch.float16)

