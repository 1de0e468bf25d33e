"""Parity and invariants at sequence lengths past the CPU oracle's reach.

The reference's longest case is its stability bench (bench/stability.py:
S up to 8192, finiteness only).  Here the kernels run at S = 12000-16384,
fwd and bwd, and are checked two ways:

* against the same attention math in float64 on the GPU (torch, a block
  of query rows at a time: scores, masked softmax, P V; then delta, dP, dS
  and the three gradients), which `test_fp64_reference_matches_oracle`
  first checks against the float64 CPU oracle at a small size, so the
  long cases carry the oracle's pinning.  Tolerance: max-abs 1e-2 on O,
  LSE, dQ, dK and dV (the suite's bar for fp16 outputs);
* by invariants that hold whatever the size and need no reference at all:
  identical keys make every output row the mean of the values its query
  sees; every output row lies between the smallest and largest visible
  value per column; max_j s_ij <= LSE_i <= max_j s_ij + ln(visible keys);
  and, since every row of P sums to one, sum_j dV_j = sum_i dO_i.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import TOL, max_abs, report
from oracle import attention as orc

pytestmark = pytest.mark.gpu

ROWS = 1024   # query rows per block of the float64 reference


def _inputs(B, Sq, Sk, H, Hk, D, seed, scale=0.5):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn((B, Sq, H, D), generator=g) * scale).half()
    k = (torch.randn((B, Sk, Hk, D), generator=g) * scale).half()
    v = (torch.randn((B, Sk, Hk, D), generator=g) * scale).half()
    do = (torch.randn((B, Sq, H, D), generator=g) * scale).half()
    return [t.cuda() for t in (q, k, v, do)]


def _heads64(t, grp):
    """(B, S, Hk, D) -> float64 (B, Hk * grp, S, D), each key/value head
    repeated for its group of query heads."""
    t = t.double().permute(0, 2, 1, 3)
    return t.repeat_interleave(grp, dim=1).contiguous() if grp > 1 else t.contiguous()


def _mask(s, r0, r1, Sk, off):
    """Causal mask of query rows [r0, r1): key j is visible to query i iff
    j <= i + off (bottom-right alignment, off = Sk - Sq)."""
    rows = torch.arange(r0, r1, device=s.device)[:, None]
    cols = torch.arange(Sk, device=s.device)[None, :]
    return s.masked_fill(cols > rows + off, -math.inf)


def ref_fwd(q, k, v, causal, scale):
    """float64 O (B, Sq, H, D) and natural-log LSE (B, H, Sq); a row that
    sees no key gets O = 0 and LSE = +inf, as the kernels give."""
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    qd, kd, vd = _heads64(q, 1), _heads64(k, H // Hk), _heads64(v, H // Hk)
    o = torch.empty((B, H, Sq, D), dtype=torch.float64, device=q.device)
    lse = torch.empty((B, H, Sq), dtype=torch.float64, device=q.device)
    for r0 in range(0, Sq, ROWS):
        r1 = min(Sq, r0 + ROWS)
        s = torch.matmul(qd[:, :, r0:r1], kd.transpose(-1, -2)) * scale
        if causal:
            s = _mask(s, r0, r1, Sk, Sk - Sq)
        m = s.amax(-1, keepdim=True)
        m0 = torch.where(torch.isinf(m), torch.zeros_like(m), m)
        p = torch.exp(s - m0)
        l = p.sum(-1, keepdim=True)
        o[:, :, r0:r1] = torch.where(l > 0, torch.matmul(p, vd) / l.clamp_min(1e-300), 0.0)
        lse[:, :, r0:r1] = torch.where(l[..., 0] > 0, (m0 + torch.log(l))[..., 0], math.inf)
    return o.permute(0, 2, 1, 3), lse


def ref_bwd(q, k, v, do, causal, scale, o, lse):
    """float64 dQ, dK, dV of L = <O, dO> given the float64 forward (o, lse);
    dK and dV summed over each key/value head's query heads."""
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    grp = H // Hk
    qd, kd, vd = _heads64(q, 1), _heads64(k, grp), _heads64(v, grp)
    dod = _heads64(do, 1)
    delta = (o.double() * do.double()).sum(-1).permute(0, 2, 1)   # (B, H, Sq)
    dq = torch.empty_like(qd)
    dk = torch.zeros_like(kd)
    dv = torch.zeros_like(vd)
    for r0 in range(0, Sq, ROWS):
        r1 = min(Sq, r0 + ROWS)
        s = torch.matmul(qd[:, :, r0:r1], kd.transpose(-1, -2)) * scale
        if causal:
            s = _mask(s, r0, r1, Sk, Sk - Sq)
        p = torch.exp(s - lse[:, :, r0:r1, None])
        dv += torch.matmul(p.transpose(-1, -2), dod[:, :, r0:r1])
        dp = torch.matmul(dod[:, :, r0:r1], vd.transpose(-1, -2))
        ds = p * (dp - delta[:, :, r0:r1, None])
        dq[:, :, r0:r1] = torch.matmul(ds, kd) * scale
        dk += torch.matmul(ds.transpose(-1, -2), qd[:, :, r0:r1]) * scale
    fold = lambda t: t.view(B, Hk, grp, Sk, D).sum(2).permute(0, 2, 1, 3)
    return dq.permute(0, 2, 1, 3), fold(dk), fold(dv)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 300, 300, 2, 2, 64), (2, 200, 333, 4, 2, 32)])
def test_fp64_reference_matches_oracle(shape, causal):
    """The float64 GPU reference restates the CPU oracle: agreement to
    rounding at a size the oracle runs in a moment (Sq < Sk included)."""
    B, Sq, Sk, H, Hk, D = shape
    print(f"[case] fp64 reference vs oracle {shape} causal={causal}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hk, D, seed=5, scale=1.0)
    sc = D ** -0.5
    o, lse = ref_fwd(q, k, v, causal, sc)
    dq, dk, dv = ref_bwd(q, k, v, do, causal, sc, o, lse)
    qc, kc, vc, doc = (t.cpu() for t in (q, k, v, do))
    o_r, l_r = orc.attention_fwd_gqa(qc, kc, vc, causal, sc)
    dq_r, dk_r, dv_r, _ = orc.attention_bwd_gqa(doc, qc, kc, vc, causal, sc, o=o_r)
    fin = np.isfinite(l_r)
    assert np.array_equal(np.isfinite(lse.cpu().numpy()), fin)
    assert float(np.abs(lse.cpu().numpy()[fin] - l_r[fin]).max()) < 1e-10
    for got, ref in ((o, o_r), (dq, dq_r), (dk, dk_r), (dv, dv_r)):
        assert max_abs(got, ref) < 1e-10


LONG = [
    # B, Sq, Sk, H, Hk, D, causal
    (1, 16384, 16384, 2, 2, 64, True),
    (1, 16384, 16384, 2, 2, 128, True),
    (1, 12000, 12000, 2, 2, 64, False),     # ragged: 12000 = 187.5 key tiles
    (1, 16384, 16384, 4, 1, 128, True),     # multi-query
    (1, 6000, 16384, 4, 2, 64, True),       # a prefill continuing a long cache
]


def _ids(c):
    B, Sq, Sk, H, Hk, D, causal = c
    return f"{B}x{Sq}x{Sk}h{H}/{Hk}d{D}{'c' if causal else 'n'}"


@pytest.mark.parametrize("case", LONG, ids=[_ids(c) for c in LONG])
def test_long_sequence_parity(case):
    from flash_attn_volta import flash_attn_forward_gqa, flash_attn_gqa
    B, Sq, Sk, H, Hk, D, causal = case
    print(f"[case] long {_ids(case)}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hk, D, seed=11)
    sc = D ** -0.5
    out, lse = flash_attn_forward_gqa(q, k, v, causal=causal, return_softmax_lse=True)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    out2 = flash_attn_gqa(qg, kg, vg, causal=causal)
    out2.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(out, out2.detach())
    o_r, l_r = ref_fwd(q, k, v, causal, sc)
    dq_r, dk_r, dv_r = ref_bwd(q, k, v, do, causal, sc, o_r, l_r)
    errs = dict(out=(out.double() - o_r).abs().max().item(),
                lse=(lse.double() - l_r).abs().max().item(),
                dq=(qg.grad.double() - dq_r).abs().max().item(),
                dk=(kg.grad.double() - dk_r).abs().max().item(),
                dv=(vg.grad.double() - dv_r).abs().max().item())
    report(f"long {_ids(case)}", **errs)
    for key, e in errs.items():
        assert e < TOL, f"{_ids(case)} {key} max-abs {e:.3e} >= {TOL}"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_identical_keys_give_means_of_visible_values(D, causal):
    """All keys equal: every score of a row is the same, P is uniform over
    the visible keys, O_i is the mean of those values and LSE_i = s_i +
    ln(visible keys) -- a prefix mean per row when causal."""
    from flash_attn_volta import flash_attn_forward
    B, S, H = 1, 16384, 2
    print(f"[case] identical keys S={S} D={D} causal={causal}", flush=True)
    q, k, v, _ = _inputs(B, S, S, H, H, D, seed=21)
    k = k[:, :1].expand(B, S, H, D).contiguous()
    out, lse = flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)
    vd = v.double()
    n = torch.arange(1, S + 1, device=v.device, dtype=torch.float64)
    mean = (vd.cumsum(1) / n[None, :, None, None]) if causal else vd.mean(1, keepdim=True)
    s = (q.double() * k.double()).sum(-1).permute(0, 2, 1) * D ** -0.5   # (B, H, S)
    lse_ref = s + (torch.log(n)[None, None] if causal else math.log(S))
    e_o = (out.double() - mean).abs().max().item()
    e_l = (lse.double() - lse_ref).abs().max().item()
    report(f"same-keys d{D}{'c' if causal else 'n'}", out=e_o, lse=e_l)
    # O: one fp16 rounding of a value <= max|v| ~ 2.5 (ulp 2^-9) plus the
    # fp32 sums; LSE: the fp16 rounding of the pre-scaled query (|s| <= ~4)
    assert e_o < 2e-3 and e_l < 5e-3


@pytest.mark.parametrize("causal", [False, True])
def test_rows_in_value_hull_and_lse_bounds(causal):
    """Rows of P are probabilities: every O_i lies between the smallest and
    largest value its query sees, per column (up to O's fp16 rounding), and
    max_j s_ij <= LSE_i <= max_j s_ij + ln(visible keys)."""
    from flash_attn_volta import flash_attn_forward
    B, S, H, D = 1, 16384, 2, 64
    print(f"[case] hull / LSE bounds S={S} causal={causal}", flush=True)
    q, k, v, _ = _inputs(B, S, S, H, H, D, seed=31, scale=1.0)
    out, lse = flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)
    vd, od = v.double(), out.double()
    if causal:
        lo, hi = vd.cummin(1).values, vd.cummax(1).values
    else:
        lo, hi = vd.amin(1, keepdim=True), vd.amax(1, keepdim=True)
    slack = 2.0 ** -10 * od.abs() + 1e-6   # O's fp16 rounding
    assert bool((od >= lo - slack).all()) and bool((od <= hi + slack).all())
    qd, kd = _heads64(q, 1), _heads64(k, 1)
    smax = torch.empty((B, H, S), dtype=torch.float64, device=q.device)
    for r0 in range(0, S, ROWS):
        s = torch.matmul(qd[:, :, r0:r0 + ROWS], kd.transpose(-1, -2)) * D ** -0.5
        if causal:
            s = _mask(s, r0, r0 + ROWS, S, 0)
        smax[:, :, r0:r0 + ROWS] = s.amax(-1)
    nvis = torch.arange(1, S + 1, device=q.device, dtype=torch.float64) if causal else S
    ld = lse.double()
    tol = TOL   # the kernels' fp16-rounded, pre-scaled queries move s by <= ~3e-3
    assert bool((ld >= smax - tol).all())
    assert bool((ld <= smax + torch.log(torch.as_tensor(nvis, dtype=torch.float64)) + tol).all())


@pytest.mark.parametrize("causal", [False, True])
def test_dv_column_sums_equal_dout_column_sums(causal):
    """dV_j = sum_i P_ij dO_i and every row of P sums to one, so
    sum_j dV_j = sum_i dO_i per (head, column).  The kernels round P to
    fp16, so row i of the P they use sums to 1 + r_i with |r_i| <= 2^-10,
    and round dV to fp16.  The r_i are sums of independent roundings, so
    sum_i dO_i r_i is of the order of 2^-10 ||dO||_2, not 2^-10 ||dO||_1:
    the two sides must agree within 2^-10 (||dO||_2 + ||dV||_2) per column
    (measured: 30-70 times inside it), tight enough that a key tile left
    out or a mis-normalised row shows."""
    from flash_attn_volta import flash_attn
    B, S, H, D = 1, 16384, 2, 128
    print(f"[case] dV column sums S={S} causal={causal}", flush=True)
    q, k, v, do = _inputs(B, S, S, H, H, D, seed=41)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    flash_attn(qg, kg, vg, causal=causal).backward(do)
    dv, dod = vg.grad.double(), do.double()
    diff = (dv.sum(1) - dod.sum(1)).abs()
    bound = 2.0 ** -10 * (dod.norm(dim=1) + dv.norm(dim=1))
    report(f"dV sums {'c' if causal else 'n'}", diff=diff.max().item(), bound=bound.min().item())
    assert bool((diff <= bound).all())
