"""Pin the grouped-query oracle functions (attention_fwd_gqa / attention_bwd_gqa)
before they check the GPU's fa_fwd_gqa / fa_bwd_gqa.

Three independent anchors:
  * golden vectors from torch's float64 scaled_dot_product_attention with
    enable_gqa and an explicit bottom-right boolean mask, and its autograd
    (tests/golden/make_golden.py, a library routine that shares no code with
    oracle/);
  * reduction identities to the already-pinned square functions
    (attention_fwd / attention_bwd): grouped heads equal attention over
    repeat_kv-expanded K/V with dK/dV summed per group; Sq < Sk equals the
    last Sq rows of a square causal problem; Sq > Sk gives empty rows
    followed by a square causal problem;
  * planted mistakes (head h -> h % Hk instead of h // group, a top-left
    instead of bottom-right causal mask) that these checks catch.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import attention as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_gqa_golden.npz")


def _cases():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, sorted({k.split("/")[0] for k in z.files})


def _case(z, name):
    g = {k.split("/")[1]: z[k] for k in z.files if k.startswith(name + "/")}
    B, Sq, Sk, H, Hk, D, causal, scale, seed = g["meta"]
    return g, bool(causal), float(scale)


@pytest.mark.parametrize("name", _cases()[1])
def test_gqa_fwd_matches_golden(name):
    z, _ = _cases()
    g, causal, scale = _case(z, name)
    o, lse = orc.attention_fwd_gqa(g["q"], g["k"], g["v"], causal, scale)
    assert o.shape == g["o"].shape and lse.shape == g["lse"].shape
    assert np.max(np.abs(o - g["o"])) < 1e-12
    assert np.max(np.abs(lse - g["lse"])) < 1e-12


@pytest.mark.parametrize("name", _cases()[1])
def test_gqa_bwd_matches_golden(name):
    z, _ = _cases()
    g, causal, scale = _case(z, name)
    dq, dk, dv, _ = orc.attention_bwd_gqa(g["do"], g["q"], g["k"], g["v"], causal, scale)
    for mine, ref in ((dq, g["dq"]), (dk, g["dk"]), (dv, g["dv"])):
        assert mine.shape == ref.shape
        assert np.max(np.abs(mine - ref)) < 1e-10


def _repeat_kv(x, grp):
    """(B, S, Hk, D) -> (B, S, Hk * grp, D), each head repeated grp times in a
    row (HuggingFace repeat_kv order)."""
    return np.repeat(np.asarray(x, dtype=np.float64), grp, axis=2)


@pytest.mark.parametrize("H,Hk", [(6, 2), (6, 3), (4, 1), (3, 3)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_equals_attention_over_repeated_heads(H, Hk, causal):
    q, k, v, do = orc.make_inputs_gqa(2, 37, 37, H, Hk, 16, seed=21)
    grp = H // Hk
    o, lse = orc.attention_fwd_gqa(q, k, v, causal)
    o2, lse2 = orc.attention_fwd(q, _repeat_kv(k, grp), _repeat_kv(v, grp), causal)
    assert np.max(np.abs(o - o2)) < 1e-12 and np.max(np.abs(lse - lse2)) < 1e-12
    dq, dk, dv, dl = orc.attention_bwd_gqa(do, q, k, v, causal)
    dq2, dk2, dv2, dl2 = orc.attention_bwd(do, q, _repeat_kv(k, grp), _repeat_kv(v, grp), causal)
    B, S = dk.shape[:2]
    assert np.max(np.abs(dq - dq2)) < 1e-12 and np.max(np.abs(dl - dl2)) < 1e-12
    assert np.max(np.abs(dk - dk2.reshape(B, S, Hk, grp, -1).sum(3))) < 1e-12
    assert np.max(np.abs(dv - dv2.reshape(B, S, Hk, grp, -1).sum(3))) < 1e-12


@pytest.mark.parametrize("Sq,Sk", [(1, 50), (13, 50), (49, 50)])
def test_bottom_right_causal_is_suffix_of_square(Sq, Sk):
    """Queries that are the last Sq positions of an Sk-long sequence: the
    rectangular causal problem is the last Sq rows of the square one."""
    B, H, D = 1, 2, 16
    qf, k, v, dof = orc.make_inputs(B, Sk, H, D, seed=22)
    q, do = qf[:, Sk - Sq:], dof[:, Sk - Sq:]
    o, lse = orc.attention_fwd_gqa(q, k, v, True)
    of, lsef = orc.attention_fwd(qf, k, v, True)
    assert np.max(np.abs(o - of[:, Sk - Sq:])) < 1e-12
    assert np.max(np.abs(lse - lsef[:, :, Sk - Sq:])) < 1e-12
    dof = dof.clone()
    dof[:, :Sk - Sq] = 0
    dq, dk, dv, _ = orc.attention_bwd_gqa(do, q, k, v, True)
    dqf, dkf, dvf, _ = orc.attention_bwd(dof, qf, k, v, True)
    assert np.max(np.abs(dq - dqf[:, Sk - Sq:])) < 1e-12
    assert np.max(np.abs(dk - dkf)) < 1e-12 and np.max(np.abs(dv - dvf)) < 1e-12


def test_more_queries_than_keys_gives_empty_rows_then_square():
    """Sq > Sk: query i sees keys j <= i - (Sq - Sk); the first Sq - Sk rows
    see nothing (o = 0, lse = +inf, no gradient), the rest are the square
    causal problem over the last Sk queries."""
    B, Sq, Sk, H, D = 1, 30, 12, 2, 16
    q, k, v, do = orc.make_inputs_gqa(B, Sq, Sk, H, H, D, seed=23)
    o, lse = orc.attention_fwd_gqa(q, k, v, True)
    e = Sq - Sk
    assert np.all(o[:, :e] == 0) and np.all(np.isinf(lse[:, :, :e]))
    o2, lse2 = orc.attention_fwd(q[:, e:], k, v, True)
    assert np.max(np.abs(o[:, e:] - o2)) < 1e-12 and np.max(np.abs(lse[:, :, e:] - lse2)) < 1e-12
    dq, dk, dv, _ = orc.attention_bwd_gqa(do, q, k, v, True)
    dq2, dk2, dv2, _ = orc.attention_bwd(do[:, e:], q[:, e:], k, v, True)
    assert np.all(dq[:, :e] == 0)
    assert np.max(np.abs(dq[:, e:] - dq2)) < 1e-12
    assert np.max(np.abs(dk - dk2)) < 1e-12 and np.max(np.abs(dv - dv2)) < 1e-12


# ---------------------------------------------------------------------------
# planted mistakes (in a copy of the oracle's forward, on the CPU)

def _mutant_fwd(q, k, v, causal, scale, kind):
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    grp = H // Hk
    off = Sk - Sq if kind != "top_left_mask" else 0
    o = np.zeros((B, Sq, H, D))
    for b in range(B):
        for h in range(H):
            kh = h % Hk if kind == "head_modulo" else h // grp
            oh, _ = orc._fwd_head(q[b, :, h], k[b, :, kh], v[b, :, kh], scale, causal, off)
            o[b, :, h] = oh
    return o


@pytest.mark.parametrize("kind,case", [("head_modulo", "gqa_h4_hk2_causal_sq_lt_sk"),
                                       ("head_modulo", "gqa_square_causal_d128"),
                                       ("top_left_mask", "gqa_h4_hk2_causal_sq_lt_sk"),
                                       ("top_left_mask", "gqa_decode_sq1")])
def test_planted_gqa_mistakes_are_caught(kind, case):
    z, _ = _cases()
    g, causal, scale = _case(z, case)
    o_bad = _mutant_fwd(g["q"], g["k"], g["v"], causal, scale, kind)
    assert np.max(np.abs(np.nan_to_num(o_bad) - g["o"])) > 1e-2
