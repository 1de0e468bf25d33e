"""Pin the rotary / QK-norm oracle (oracle/rope.py) before it checks the GPU's
fa_rope_qk_fwd / fa_rope_qk_bwd.

Anchors:
  * golden vectors from transformers' own apply_rotary_pos_emb and
    Qwen3RMSNorm in float64 with torch autograd for the gradients
    (tests/golden/make_rope_golden.py).  Qwen3RMSNorm computes its
    statistics in float32 whatever the input dtype, so normed sides agree
    to ~1e-6 rather than to float64 rounding; un-normed sides are exact;
  * closed forms: position 0 is the identity, rotation keeps each (d, d+D/2)
    pair's norm, rotating by -theta undoes +theta, unit-weight RMSNorm
    output has mean square 1 (eps = 0);
  * central finite differences of rope_qk_fwd and the adjoint identity;
  * planted mistakes (interleaved pairs, the opposite rotation sign, a norm
    that drops its weight) that these checks catch.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import rope as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rope_golden.npz")


def _cases():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, sorted({k.split("/")[0] for k in z.files})


def _case(name):
    z, _ = _cases()
    g = {k.split("/")[1]: z[k] for k in z.files if k.startswith(name + "/")}
    return g, float(g["meta"][7])


def _tol(w):
    # transformers' RMSNorm keeps its statistics in float32
    return 1e-12 if w is None else 5e-6


@pytest.mark.parametrize("name", _cases()[1])
def test_rope_fwd_matches_golden(name):
    g, eps = _case(name)
    wq, wk = g.get("wq"), g.get("wk")
    qo, ko = orc.rope_qk_fwd(g["q"], g["k"], g["cos"], g["sin"], wq, wk, eps)
    assert qo.shape == g["q_out"].shape and ko.shape == g["k_out"].shape
    assert np.max(np.abs(qo - g["q_out"])) < _tol(wq)
    assert np.max(np.abs(ko - g["k_out"])) < _tol(wk)


@pytest.mark.parametrize("name", _cases()[1])
def test_rope_bwd_matches_golden(name):
    g, eps = _case(name)
    wq, wk = g.get("wq"), g.get("wk")
    dq, dk, dwq, dwk = orc.rope_qk_bwd(g["dq_out"], g["dk_out"], g["q"], g["k"], g["cos"],
                                       g["sin"], wq, wk, eps)
    assert np.max(np.abs(dq - g["dq"])) < _tol(wq)
    assert np.max(np.abs(dk - g["dk"])) < _tol(wk)
    assert (dwq is None) == (wq is None) and (dwk is None) == (wk is None)
    if wq is not None:
        assert np.max(np.abs(dwq - g["dwq"])) < 1e-5 * max(1.0, np.abs(g["dwq"]).max())
    if wk is not None:
        assert np.max(np.abs(dwk - g["dwk"])) < 1e-5 * max(1.0, np.abs(g["dwk"]).max())


def test_position_zero_is_identity():
    q, k, cos, sin, *_ = orc.make_rope_inputs(1, 6, 2, 1, 64, seed=5)
    qo, ko = orc.rope_qk_fwd(q, k, cos, sin)
    assert np.array_equal(qo[:, 0], q[:, 0].double().numpy())
    assert np.array_equal(ko[:, 0], k[:, 0].double().numpy())
    assert not np.allclose(qo[:, 1:], q[:, 1:].double().numpy())


def test_rotation_keeps_pair_norms_and_inverts():
    B, S, H, D = 2, 11, 3, 32
    q, k, _, _, *_ = orc.make_rope_inputs(B, S, H, H, D, seed=6)
    theta = np.random.default_rng(0).uniform(-7, 7, size=(B, S, D // 2))
    theta = np.concatenate([theta, theta], axis=-1)   # transformers' emb = cat(freqs, freqs)
    c, s = np.cos(theta), np.sin(theta)
    qo, _ = orc.rope_qk_fwd(q, k, c, s)
    x = q.double().numpy()
    h = D // 2
    assert np.allclose(qo[..., :h] ** 2 + qo[..., h:] ** 2, x[..., :h] ** 2 + x[..., h:] ** 2,
                       atol=1e-12)
    back, _ = orc.rope_qk_fwd(qo, k, c, -s)
    assert np.max(np.abs(back - x)) < 1e-12


def test_unit_weight_norm_has_unit_mean_square():
    q, k, cos, sin, *_ = orc.make_rope_inputs(1, 4, 2, 2, 64, seed=7, shared_table=True)
    w = np.ones(64)
    ones, zeros = np.ones((1, 4, 64)), np.zeros((1, 4, 64))
    qo, ko = orc.rope_qk_fwd(q, k, ones, zeros, w, w, eps=0.0)
    assert np.allclose(np.mean(qo ** 2, axis=-1), 1.0, atol=1e-12)
    assert np.allclose(np.mean(ko ** 2, axis=-1), 1.0, atol=1e-12)
    # scale invariance of the normed side
    qo2, _ = orc.rope_qk_fwd(q.double() * 3.0, k, ones, zeros, w, w, eps=0.0)
    assert np.max(np.abs(qo2 - qo)) < 1e-12


@pytest.mark.parametrize("norm", [False, True])
def test_bwd_matches_finite_differences(norm):
    B, S, H, Hk, D = 1, 3, 2, 1, 16
    q, k, cos, sin, wq, wk, gq, gk = orc.make_rope_inputs(B, S, H, Hk, D, seed=8, norm=True)
    if not norm:
        wq = wk = None
    eps = 1e-3
    x = [q.double().numpy().copy(), k.double().numpy().copy()]
    w = [None if wq is None else wq.double().numpy().copy(),
         None if wk is None else wk.double().numpy().copy()]
    g = [gq.double().numpy(), gk.double().numpy()]

    def loss():
        qo, ko = orc.rope_qk_fwd(x[0], x[1], cos, sin, w[0], w[1], eps)
        return float(np.sum(qo * g[0]) + np.sum(ko * g[1]))

    dq, dk, dwq, dwk = orc.rope_qk_bwd(gq, gk, x[0], x[1], cos, sin, w[0], w[1], eps)
    h = 1e-6
    targets = [(x[0], dq), (x[1], dk)]
    if norm:
        targets += [(w[0], dwq), (w[1], dwk)]
    for arr, grad in targets:
        flat, gflat = arr.reshape(-1), grad.reshape(-1)
        for i in range(0, flat.size, max(1, flat.size // 23)):
            old = flat[i]
            flat[i] = old + h
            lp = loss()
            flat[i] = old - h
            lm = loss()
            flat[i] = old
            assert abs((lp - lm) / (2 * h) - gflat[i]) < 1e-6 * max(1.0, abs(gflat[i]))


def test_adjoint_identity():
    B, S, H, D = 2, 5, 3, 64
    q, k, cos, sin, _, _, gq, gk = orc.make_rope_inputs(B, S, H, H, D, seed=9)
    qo, _ = orc.rope_qk_fwd(q, k, cos, sin)
    dq, _, _, _ = orc.rope_qk_bwd(gq, gk, q, k, cos, sin)
    lhs = np.sum(qo * gq.double().numpy())
    rhs = np.sum(q.double().numpy() * dq)
    assert abs(lhs - rhs) < 1e-9 * max(1.0, abs(lhs))


# ---------------------------------------------------------------------------
# planted mistakes (in copies of the oracle's forward, on the CPU)

def _mutant(x, c, s, w, eps, kind):
    x = np.asarray(x, dtype=np.float64)
    c, s = c[:, :, None, :], s[:, :, None, :]
    y = x
    if w is not None:
        n = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
        y = n if kind == "norm_without_weight" else n * w
    if kind == "interleaved":
        r = np.empty_like(y)
        r[..., 0::2], r[..., 1::2] = -y[..., 1::2], y[..., 0::2]
    else:
        h = y.shape[-1] // 2
        r = np.concatenate([-y[..., h:], y[..., :h]], axis=-1)
        if kind == "opposite_sign":
            r = -r
    return y * c + r * s


@pytest.mark.parametrize("kind,case", [("interleaved", "llama_gqa_d64"),
                                       ("opposite_sign", "qwen3_mqa_d128"),
                                       ("norm_without_weight", "qwen3_d16_far")])
def test_planted_rope_mistakes_are_caught(kind, case):
    g, eps = _case(case)
    bad = _mutant(g["q"], g["cos"].astype(np.float64), g["sin"].astype(np.float64), g.get("wq"),
                  eps, kind)
    assert np.max(np.abs(bad - g["q_out"])) > 1e-2
