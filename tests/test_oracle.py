"""Pin the CPU oracle (oracle/) before trusting it as the parity checker.

Every oracle function is checked against something that does not share its
code: torch float64 SDPA/autograd golden vectors (tests/golden/), the
plain-C brute force (oracle/attention_ref.c), closed-form special cases, and
central finite differences of the forward.  The planted-mistake tests show
these checks fail for plausible oracle bugs (a dropped scale, a transposed
product, a wrong delta, a shifted causal diagonal).
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as orc
from oracle import build as orc_build

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz")


def _golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def _case(z, name):
    g = {k.split("/")[1]: z[k] for k in z.files if k.startswith(name + "/")}
    B, S, H, D, causal, scale, seed = g["meta"]
    return g, bool(causal), float(scale)


@pytest.mark.parametrize("name", _golden_cases()[1])
def test_fwd_matches_golden(name):
    z, _ = _golden_cases()
    g, causal, scale = _case(z, name)
    o, lse = orc.attention_fwd(g["q"], g["k"], g["v"], causal, scale)
    assert np.max(np.abs(o - g["o"])) < 1e-12
    assert np.max(np.abs(lse - g["lse"])) < 1e-12


@pytest.mark.parametrize("name", _golden_cases()[1])
def test_bwd_matches_golden(name):
    z, _ = _golden_cases()
    g, causal, scale = _case(z, name)
    dq, dk, dv, _ = orc.attention_bwd(g["do"], g["q"], g["k"], g["v"], causal, scale)
    for mine, ref in ((dq, g["dq"]), (dk, g["dk"]), (dv, g["dv"])):
        assert np.max(np.abs(mine - ref)) < 1e-10


# ---------------------------------------------------------------------------
# C brute force vs numpy oracle

def _c_fwd_bwd(q, k, v, do, causal, scale, o_given=None):
    lib = orc_build.load()
    q, k, v, do = (np.ascontiguousarray(np.asarray(t, np.float64)) for t in (q, k, v, do))
    B, S, H, D = q.shape
    P = ctypes.POINTER(ctypes.c_double)
    ptr = lambda a: a.ctypes.data_as(P)  # noqa: E731
    o = np.zeros_like(q)
    lse = np.zeros((B, H, S))
    assert lib.oracle_fwd(ptr(q), ptr(k), ptr(v), B, S, H, D, scale, int(causal), ptr(o), ptr(lse)) == 0
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    delta = np.zeros((B, H, S))
    og = None if o_given is None else np.ascontiguousarray(np.asarray(o_given, np.float64))
    assert lib.oracle_bwd(ptr(do), ptr(q), ptr(k), ptr(v), ptr(og) if og is not None else None,
                          B, S, H, D, scale, int(causal), ptr(dq), ptr(dk), ptr(dv), ptr(delta)) == 0
    return o, lse, dq, dk, dv, delta


@pytest.mark.parametrize("shape,causal,scale", [
    ((1, 7, 1, 8), False, None),
    ((2, 19, 3, 16), True, None),
    ((1, 33, 2, 32), True, 0.3),
    ((1, 24, 2, 64), False, -0.2),
    ((1, 9, 1, 128), True, 0.0),
])
def test_c_oracle_matches_numpy(shape, causal, scale):
    B, S, H, D = shape
    q, k, v, do = (t.numpy() for t in orc.make_inputs(B, S, H, D, seed=11))
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    o, lse = orc.attention_fwd(q, k, v, causal, sc)
    dq, dk, dv, delta = orc.attention_bwd(do, q, k, v, causal, sc)
    co, clse, cdq, cdk, cdv, cdelta = _c_fwd_bwd(q, k, v, do, causal, sc)
    for a, b in ((o, co), (lse, clse), (dq, cdq), (dk, cdk), (dv, cdv), (delta, cdelta)):
        assert np.max(np.abs(a - b)) < 1e-10


def test_c_oracle_uses_given_o_for_delta():
    q, k, v, do = (t.numpy() for t in orc.make_inputs(1, 12, 1, 32, seed=3))
    o, _ = orc.attention_fwd(q, k, v, True, 0.2)
    o16 = o.astype(np.float16)
    delta_np = orc.attention_bwd(do, q, k, v, True, 0.2, o=o16)[3]
    delta_c = _c_fwd_bwd(q, k, v, do, True, 0.2, o_given=o16)[5]
    assert np.max(np.abs(delta_np - delta_c)) < 1e-12
    expect = (o16.astype(np.float64) * do.astype(np.float64)).sum(-1).transpose(0, 2, 1)
    assert np.max(np.abs(delta_np - expect)) < 1e-12


# ---------------------------------------------------------------------------
# closed forms

def test_single_key_returns_v_and_dot_lse():
    q, k, v, _ = (t.numpy().astype(np.float64) for t in orc.make_inputs(2, 1, 3, 64, seed=5))
    o, lse = orc.attention_fwd(q, k, v, False, 0.125)
    assert np.array_equal(o, v)
    expect = 0.125 * np.einsum("bshd,bshd->bhs", q, k)
    assert np.max(np.abs(lse - expect)) < 1e-12


def test_causal_first_row():
    q, k, v, _ = (t.numpy().astype(np.float64) for t in orc.make_inputs(1, 20, 2, 32, seed=6))
    o, lse = orc.attention_fwd(q, k, v, True, 0.5)
    assert np.max(np.abs(o[:, 0] - v[:, 0])) < 1e-15
    assert np.max(np.abs(lse[:, :, 0] - 0.5 * np.einsum("bhd,bhd->bh", q[:, 0], k[:, 0]))) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_identical_keys_average_values(causal):
    B, S, H, D = 1, 17, 2, 16
    q, _, v, _ = (t.numpy().astype(np.float64) for t in orc.make_inputs(B, S, H, D, seed=7))
    k = np.broadcast_to(np.random.default_rng(0).standard_normal((1, 1, H, D)), (B, S, H, D)).copy()
    o, lse = orc.attention_fwd(q, k, v, causal, 0.3)
    for i in range(S):
        n = i + 1 if causal else S
        assert np.max(np.abs(o[:, i] - v[:, :n].mean(axis=1))) < 1e-12
        s = 0.3 * np.einsum("bhd,bhd->bh", q[:, i], k[:, 0])
        assert np.max(np.abs(lse[:, :, i] - (s + math.log(n)))) < 1e-12


def test_zero_scale_is_uniform_average():
    q, k, v, _ = (t.numpy().astype(np.float64) for t in orc.make_inputs(1, 9, 1, 32, seed=8))
    o, lse = orc.attention_fwd(q, k, v, False, 0.0)
    assert np.max(np.abs(o - v.mean(axis=1, keepdims=True))) < 1e-12
    assert np.max(np.abs(lse - math.log(9))) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_convex_hull_and_lse_bounds(causal):
    B, S, H, D = 2, 30, 2, 32
    q, k, v, _ = (t.numpy().astype(np.float64) for t in orc.make_inputs(B, S, H, D, seed=9))
    o, lse = orc.attention_fwd(q, k, v, causal, 0.25)
    for i in range(S):
        n = i + 1 if causal else S
        vis = v[:, :n]
        assert np.all(o[:, i] <= vis.max(axis=1) + 1e-12)
        assert np.all(o[:, i] >= vis.min(axis=1) - 1e-12)
        s = 0.25 * np.einsum("bhd,bjhd->bhj", q[:, i], k[:, :n])
        assert np.all(lse[:, :, i] >= s.max(-1) - 1e-12)
        assert np.all(lse[:, :, i] <= s.max(-1) + math.log(n) + 1e-12)


# ---------------------------------------------------------------------------
# finite differences of the forward pin the backward formulas

def _fd_grads(q, k, v, do, causal, scale, eps=1e-6):
    def loss(qq, kk, vv):
        return float((orc.attention_fwd(qq, kk, vv, causal, scale)[0] * do).sum())
    grads = []
    for which in range(3):
        args = [q.copy(), k.copy(), v.copy()]
        g = np.zeros_like(args[which])
        it = np.nditer(g, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            g[idx] = (loss(*plus) - loss(*minus)) / (2 * eps)
        grads.append(g)
    return grads


def _fd_case(causal):
    q, k, v, do = (t.numpy().astype(np.float64) for t in orc.make_inputs(1, 6, 2, 4, seed=12))
    return q, k, v, do, causal, 0.7


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_matches_finite_differences(causal):
    q, k, v, do, causal, scale = _fd_case(causal)
    fd = _fd_grads(q, k, v, do, causal, scale)
    an = orc.attention_bwd(do, q, k, v, causal, scale)[:3]
    for a, f in zip(an, fd):
        assert np.max(np.abs(a - f)) < 1e-7


# Planted mistakes: each mutant oracle must FAIL the same checks.
def _mutant_bwd(kind, do, q, k, v, causal, scale):
    dq, dk, dv, delta = orc.attention_bwd(do, q, k, v, causal, scale)
    if kind == "dk_no_scale":
        dk = dk / scale
    elif kind == "dv_untransposed":
        B, S, H, D = q.shape
        o, lse = orc.attention_fwd(q, k, v, causal, scale)
        for b in range(B):
            for h in range(H):
                s = orc._scores(q[b, :, h], k[b, :, h], scale, causal)
                p = np.exp(s - lse[b, h][:, None])
                dv[b, :, h] = p @ do[b, :, h]
    elif kind == "delta_zero":
        dq2, dk2, dv2, _ = orc.attention_bwd(do, q, k, v, causal, scale, o=np.zeros_like(q))
        dq, dk = dq2, dk2
    elif kind == "dq_sign":
        dq = -dq
    return dq, dk, dv


@pytest.mark.parametrize("kind", ["dk_no_scale", "dv_untransposed", "delta_zero", "dq_sign"])
def test_planted_backward_mistake_is_caught(kind):
    q, k, v, do, causal, scale = _fd_case(True)
    fd = _fd_grads(q, k, v, do, causal, scale)
    an = _mutant_bwd(kind, do, q, k, v, causal, scale)
    worst = max(np.max(np.abs(a - f)) for a, f in zip(an, fd))
    assert worst > 1e-3, f"mutant {kind} not detected (worst {worst:.2e})"


def test_planted_causal_diagonal_mistake_is_caught():
    """A mask that also hides the diagonal (triu k=0) must disagree with the
    golden vectors."""
    z, _ = _golden_cases()
    g, causal, scale = _case(z, "tiny_causal_d32")
    q, k, v = (g[x].astype(np.float64) for x in ("q", "k", "v"))
    s = np.einsum("bihd,bjhd->bhij", q, k) * scale
    S = s.shape[-1]
    s[..., np.triu_indices(S, k=0)[0], np.triu_indices(S, k=0)[1]] = -np.inf
    with np.errstate(invalid="ignore"):
        m = np.max(s, -1, keepdims=True)
        p = np.exp(s - m)
        p = p / p.sum(-1, keepdims=True)
    o_bad = np.einsum("bhij,bjhd->bihd", np.nan_to_num(p), v)
    assert np.nanmax(np.abs(o_bad - g["o"])) > 1e-2


# ---------------------------------------------------------------------------
# the fp32 CPU path (reference ref.py restated) agrees with the fp64 oracle

@pytest.mark.parametrize("causal", [False, True])
def test_ref_fp32_matches_oracle(causal):
    q, k, v, _ = orc.make_inputs(2, 64, 2, 64, seed=13)
    out = orc.attention_ref_fp32(q, k, v, causal)
    o, _ = orc.attention_fwd(q, k, v, causal)
    assert out.dtype == torch.float16
    assert np.max(np.abs(out.double().numpy() - o)) < 2e-3


def test_make_inputs_is_deterministic():
    a = orc.make_inputs(1, 8, 2, 32, seed=4)
    b = orc.make_inputs(1, 8, 2, 32, seed=4)
    for x, y in zip(a, b):
        assert torch.equal(x, y) and x.dtype == torch.float16
    q, k, v, do = a
    assert not torch.equal(q, k) and not torch.equal(q, do)
