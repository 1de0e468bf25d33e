"""Seeded sweep of random shapes through the grouped-query entry points
(flash_attn_forward_gqa / flash_attn_backward_gqa) against float32
attention and autograd in torch on the same GPU.

The BASELINE configs and the edge cases have tests of their own against the
float64 oracle; this sweep covers the combinations between them: ragged
query and key lengths (Sq != Sk, bottom-right causal), grouped heads, every
native head dim, fp16 and bf16, signed scales and (B, H, S, D) views passed
in place.  Each case prints its parameters before it runs.  Tolerances as
in the rest of the suite: max-abs 1e-2 for fp16 outputs, 4e-2 for bf16.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import TOL

pytestmark = pytest.mark.gpu

N_CASES = 24


def _case(i: int) -> dict:
    r = np.random.RandomState(1000 + i)
    D = int(r.choice([32, 64, 128]))
    Hk = int(r.choice([1, 2, 4]))
    H = Hk * int(r.choice([1, 2, 4]))
    causal = bool(r.rand() < 0.6)
    Sq = int(r.randint(1, 600))
    # causal masks are bottom-right aligned: keep every query row's key
    # range non-empty (Sk >= Sq)
    Sk = int(r.randint(Sq, 700)) if causal else int(r.randint(1, 700))
    if r.rand() < 0.3:
        Sk = Sq
    return dict(B=int(r.randint(1, 3)), Sq=Sq, Sk=Sk, H=H, Hk=Hk, D=D, causal=causal,
                dtype=torch.bfloat16 if r.rand() < 0.3 else torch.float16,
                # around the default 1/sqrt(D), signed: the absolute
                # tolerances hold for gradients of that size (at 3.4x the
                # default, D = 128, |dK| reaches ~15 and its fp16 error
                # 2e-2, 0.14 % of it)
                sm_scale=[None, 0.5 / math.sqrt(D), -1.0 / math.sqrt(D),
                          1.5 / math.sqrt(D)][int(r.randint(0, 4))],
                views=bool(r.rand() < 0.3), seed=2000 + i)


def _inputs(c: dict):
    g = torch.Generator("cpu").manual_seed(c["seed"])
    B, Sq, Sk, H, Hk, D = (c[k] for k in ("B", "Sq", "Sk", "H", "Hk", "D"))

    def make(S, heads):
        x = torch.randn(B, heads, S, D, generator=g).to(c["dtype"]).cuda()
        # a (B, H, S, D) tensor seen as (B, S, H, D): strides not contiguous
        return x.transpose(1, 2) if c["views"] else x.transpose(1, 2).contiguous()

    return make(Sq, H), make(Sk, Hk), make(Sk, Hk), make(Sq, H)


def _reference(q, k, v, do, causal, sc):
    """float32 attention and gradients, (B, S, H, D) in and out."""
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    qf, kf, vf = (t.float().permute(0, 2, 1, 3).contiguous().requires_grad_() for t in (q, k, v))
    ke = kf.repeat_interleave(H // Hk, dim=1)
    ve = vf.repeat_interleave(H // Hk, dim=1)
    s = torch.matmul(qf, ke.transpose(-1, -2).contiguous()) * sc
    if causal:
        i = torch.arange(Sq, device=q.device)[:, None]
        j = torch.arange(Sk, device=q.device)[None, :]
        s = s.masked_fill(j > i + (Sk - Sq), float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), ve)
    o.backward(do.float().permute(0, 2, 1, 3).contiguous())
    back = lambda t: t.permute(0, 2, 1, 3)
    return back(o.detach()), back(qf.grad), back(kf.grad), back(vf.grad)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape(i):
    from flash_attn_volta import flash_attn_backward_gqa, flash_attn_forward_gqa
    c = _case(i)
    print(f"[case] sweep {i}: " + ", ".join(f"{k}={v}" for k, v in c.items()), flush=True)
    q, k, v, do = _inputs(c)
    sc = c["sm_scale"] if c["sm_scale"] is not None else 1.0 / math.sqrt(c["D"])
    o, lse = flash_attn_forward_gqa(q, k, v, causal=c["causal"], sm_scale=c["sm_scale"],
                                    return_softmax_lse=True)
    dq, dk, dv = flash_attn_backward_gqa(do, q, k, v, o, lse, causal=c["causal"],
                                         sm_scale=c["sm_scale"])
    torch.cuda.synchronize()
    ref = _reference(q, k, v, do, c["causal"], sc)
    tol = TOL if c["dtype"] == torch.float16 else 4e-2
    for name, ours, want in zip(("o", "dq", "dk", "dv"), (o, dq, dk, dv), ref):
        assert ours.shape == want.shape and ours.dtype == c["dtype"], name
        err = float((ours.float() - want).abs().max())
        assert math.isfinite(err) and err < tol, f"{name} max-abs {err:.3e} >= {tol}"
