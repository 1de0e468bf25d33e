"""Grouped-query attention, Sq != Sk and bf16 on the GPU:
flash_attn_forward_gqa / flash_attn_backward_gqa / flash_attn_gqa
(fa_fwd_gqa / fa_bwd_gqa via the C ABI) against the float64 oracle
(attention_fwd_gqa / attention_bwd_gqa) on identical seeded 16-bit inputs.
Tolerance: max-abs 1e-2 on O, LSE and every gradient for fp16, as for the
square entry points; 4e-2 for bf16 (see BF16_TOL).

Cases: GQA and MQA groups at equal lengths; fewer queries than keys
(prefill continuation, single-token decode) and more queries than keys
(rows that see no key: O = 0, LSE = +inf, zero gradient); ragged lengths;
D = 16/32/64/128; grids large enough for the unsplit kernels; HF-layout
strided inputs; determinism; equivalence with the square entry points when
Hk == H and Sq == Sk, and with attention over repeat_kv-expanded K/V.
"""
from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from helpers import TOL, default_scale, max_abs, report
from oracle import attention as orc

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=2)
def _oracle(B, Sq, Sk, H, Hk, D, causal, seed, dtype=torch.float16):
    q, k, v, do = orc.make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=seed, dtype=dtype)
    sc = default_scale(D, None)
    o, lse = orc.attention_fwd_gqa(q, k, v, causal, sc)
    dq, dk, dv, _ = orc.attention_bwd_gqa(do, q, k, v, causal, sc, o=o)
    return (q, k, v, do), (o, lse, dq, dk, dv)


def _lse_err(lse, ref):
    """max-abs over finite entries; +inf (row with no visible key) must match
    exactly."""
    a = lse.detach().double().cpu().numpy()
    inf_ref = np.isinf(ref)
    assert np.array_equal(np.isinf(a), inf_ref), "rows with no visible key differ"
    return float(np.max(np.abs(a[~inf_ref] - ref[~inf_ref]))) if (~inf_ref).any() else 0.0


def _run(q, k, v, do, causal):
    from flash_attn_volta import flash_attn_backward_gqa, flash_attn_forward_gqa
    qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
    out, lse = flash_attn_forward_gqa(qd, kd, vd, causal=causal, return_softmax_lse=True)
    dq, dk, dv = flash_attn_backward_gqa(dod, qd, kd, vd, out, lse, causal=causal)
    torch.cuda.synchronize()
    return out, lse, dq, dk, dv


CASES = [
    # (B, Sq, Sk, H, Hk, D, causal)
    (2, 300, 300, 8, 2, 64, True),
    (2, 300, 300, 8, 2, 64, False),
    (1, 1024, 1024, 16, 4, 128, True),
    (1, 257, 257, 6, 1, 32, True),            # MQA
    (1, 100, 900, 8, 2, 64, True),            # prefill continuation
    (1, 100, 900, 8, 2, 64, False),
    (2, 1, 513, 4, 4, 128, True),             # single-token decode
    (1, 3, 1000, 8, 1, 64, True),
    (1, 64, 4096, 8, 8, 64, True),
    (1, 500, 130, 4, 2, 64, True),            # rows with no visible key
    (1, 500, 130, 4, 2, 64, False),
    (2, 77, 191, 6, 3, 32, True),             # ragged
    (1, 129, 65, 2, 1, 128, True),
    (1, 200, 333, 4, 2, 16, True),            # D = 16 (zero-padded to 32)
]


@pytest.mark.parametrize("case", CASES, ids=[
    f"B{c[0]}_q{c[1]}_k{c[2]}_H{c[3]}_Hk{c[4]}_D{c[5]}_{'c' if c[6] else 'n'}" for c in CASES])
def test_gqa_parity(case):
    B, Sq, Sk, H, Hk, D, causal = case
    print(f"[case] gqa {case}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv) = _oracle(B, Sq, Sk, H, Hk, D, causal, 31)
    out, glse, gq, gk, gv = _run(q, k, v, do, causal)
    assert out.shape == (B, Sq, H, D) and gk.shape == (B, Sk, Hk, D) and gv.shape == gk.shape
    errs = dict(out=max_abs(out, o), lse=_lse_err(glse, lse), dq=max_abs(gq, dq),
                dk=max_abs(gk, dk), dv=max_abs(gv, dv))
    report(f"gqa {Sq}x{Sk} {H}/{Hk}", **errs)
    for key, e in errs.items():
        assert e < TOL, f"{case} {key} max-abs {e:.3e} >= {TOL}"


# Grids large enough for the unsplit kernels (the last two run the eight-wave
# D = 128 dK/dV layout, grouped query heads sharing its K / V in LDS).
@pytest.mark.parametrize("case", [(4, 1000, 1000, 32, 8, 64, True), (4, 520, 777, 32, 4, 128, False),
                                  (8, 300, 700, 32, 16, 32, True), (4, 600, 1100, 32, 8, 128, False),
                                  (4, 300, 1100, 32, 16, 128, True)])
def test_gqa_large_grid_variant(case):
    B, Sq, Sk, H, Hk, D, causal = case
    print(f"[case] gqa large-grid {case}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv) = _oracle(B, Sq, Sk, H, Hk, D, causal, 32)
    out, glse, gq, gk, gv = _run(q, k, v, do, causal)
    errs = dict(out=max_abs(out, o), lse=_lse_err(glse, lse), dq=max_abs(gq, dq),
                dk=max_abs(gk, dk), dv=max_abs(gv, dv))
    report(f"gqa-large {Sq}x{Sk}", **errs)
    for key, e in errs.items():
        assert e < TOL, f"{case} {key} max-abs {e:.3e} >= {TOL}"


@pytest.mark.parametrize("causal", [False, True])
def test_gqa_with_equal_heads_and_lengths_is_the_square_path(causal):
    """Hk == H, Sq == Sk: the grouped entry points give bit-identical results
    to flash_attn_forward / flash_attn_backward."""
    from flash_attn_volta import (flash_attn_backward, flash_attn_backward_gqa, flash_attn_forward,
                                  flash_attn_forward_gqa)
    q, k, v, do = (t.cuda() for t in orc.make_inputs(2, 333, 4, 64, seed=33))
    o1, l1 = flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)
    o2, l2 = flash_attn_forward_gqa(q, k, v, causal=causal, return_softmax_lse=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    g1 = flash_attn_backward(do, q, k, v, o1, l1, causal=causal)
    g2 = flash_attn_backward_gqa(do, q, k, v, o1, l1, causal=causal)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_gqa_forward_equals_repeated_heads_bitwise():
    """Each query head reads its key/value head in place: the forward is
    bit-identical to the square kernel on repeat_kv-expanded K/V."""
    from flash_attn_volta import flash_attn_forward, flash_attn_forward_gqa
    q, k, v, _ = (t.cuda() for t in orc.make_inputs_gqa(1, 400, 400, 8, 2, 64, seed=34))
    kr, vr = (t.repeat_interleave(4, dim=2).contiguous() for t in (k, v))
    for causal in (False, True):
        a, la = flash_attn_forward_gqa(q, k, v, causal=causal, return_softmax_lse=True)
        b, lb = flash_attn_forward(q, kr, vr, causal=causal, return_softmax_lse=True)
        assert torch.equal(a, b) and torch.equal(la, lb)


def test_gqa_autograd_and_strided_inputs():
    """flash_attn_gqa through autograd on (B, H, S, D).transpose(1, 2) views
    (the HuggingFace layout) matches contiguous inputs bit for bit, and is
    deterministic run to run."""
    from flash_attn_volta import flash_attn_gqa
    q, k, v, do = orc.make_inputs_gqa(2, 190, 450, 6, 2, 64, seed=35)

    def run(strided):
        ts = []
        for t in (q, k, v):
            t = t.cuda()
            if strided:
                t = t.permute(0, 2, 1, 3).contiguous().transpose(1, 2)
            ts.append(t.requires_grad_())
        out = flash_attn_gqa(*ts, causal=True)
        out.backward(do.cuda())
        return [out.detach()] + [t.grad for t in ts]

    a, b, c = run(False), run(True), run(False)
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(x, z)


# bf16: max-abs 4e-2, four times the fp16 bar (bf16 keeps 2 fewer mantissa
# bits, so its rounding of the inputs, of P and dS, and of the outputs is 4x
# coarser).  The oracle sees the same bf16 inputs.
BF16_TOL = 4e-2
BF16_CASES = [
    (2, 300, 300, 8, 2, 64, True),
    (1, 1024, 1024, 8, 8, 128, True),
    (1, 100, 900, 8, 2, 64, False),
    (1, 500, 130, 4, 2, 64, True),
    (2, 77, 191, 6, 3, 32, True),
    (1, 200, 333, 4, 2, 16, False),
    (1, 4096, 4096, 16, 16, 64, True),        # the C4a shape
    (1, 600, 600, 64, 64, 128, False),        # grid for the eight-wave D = 128 dK/dV
    (1, 2100, 2100, 32, 8, 64, False),        # eight-wave forward (256 queries), ragged
    (1, 2100, 2100, 16, 4, 128, False),       # eight-wave key-split forward, ragged
]


@pytest.mark.parametrize("case", BF16_CASES, ids=[
    f"bf16_B{c[0]}_q{c[1]}_k{c[2]}_H{c[3]}_Hk{c[4]}_D{c[5]}_{'c' if c[6] else 'n'}" for c in BF16_CASES])
def test_gqa_bf16_parity(case):
    B, Sq, Sk, H, Hk, D, causal = case
    print(f"[case] gqa bf16 {case}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv) = _oracle(B, Sq, Sk, H, Hk, D, causal, 36, torch.bfloat16)
    out, glse, gq, gk, gv = _run(q, k, v, do, causal)
    assert out.dtype == gq.dtype == gk.dtype == gv.dtype == torch.bfloat16
    errs = dict(out=max_abs(out, o), lse=_lse_err(glse, lse), dq=max_abs(gq, dq),
                dk=max_abs(gk, dk), dv=max_abs(gv, dv))
    report(f"bf16 {Sq}x{Sk} {H}/{Hk} D{D}", **errs)
    for key, e in errs.items():
        assert e < BF16_TOL, f"{case} {key} max-abs {e:.3e} >= {BF16_TOL}"


def test_gqa_bf16_negative_and_large_scale():
    """bf16 keeps K unscaled in the dK/dV recompute, so |sm_scale| > ln 2
    and negative scales take the general exponent path."""
    from flash_attn_volta import flash_attn_backward_gqa, flash_attn_forward_gqa
    B, Sq, Sk, H, Hk, D = 1, 200, 260, 4, 2, 64
    q, k, v, do = orc.make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=37, scale=0.25, dtype=torch.bfloat16)
    for scale in (-0.125, 0.9):
        o, lse = orc.attention_fwd_gqa(q, k, v, True, scale)
        dq, dk, dv, _ = orc.attention_bwd_gqa(do, q, k, v, True, scale, o=o)
        qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
        out, glse = flash_attn_forward_gqa(qd, kd, vd, causal=True, sm_scale=scale,
                                           return_softmax_lse=True)
        gq, gk, gv = flash_attn_backward_gqa(dod, qd, kd, vd, out, glse, causal=True, sm_scale=scale)
        errs = dict(out=max_abs(out, o), lse=_lse_err(glse, lse), dq=max_abs(gq, dq),
                    dk=max_abs(gk, dk), dv=max_abs(gv, dv))
        report(f"bf16 scale {scale}", **errs)
        for key, e in errs.items():
            assert e < BF16_TOL, f"scale {scale} {key} max-abs {e:.3e}"


def test_gqa_argument_errors():
    from flash_attn_volta import flash_attn_forward_gqa
    from flash_attn_volta.forward import FlashAttnArgumentError
    q = torch.zeros(1, 8, 6, 64, dtype=torch.float16, device="cuda")
    k = torch.zeros(1, 8, 4, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(FlashAttnArgumentError):
        flash_attn_forward_gqa(q, k, k)                      # 6 % 4 != 0
    with pytest.raises(FlashAttnArgumentError):
        flash_attn_forward_gqa(q, k[..., :32], k[..., :32])  # head_dim mismatch
    with pytest.raises(FlashAttnArgumentError):
        flash_attn_forward_gqa(q, k[:, :, :2], k[:, :, :3])  # k / v differ
    with pytest.raises(FlashAttnArgumentError):
        flash_attn_forward_gqa(q.bfloat16(), k[:, :, :2], k[:, :, :2])   # mixed dtypes
    with pytest.raises(FlashAttnArgumentError):
        flash_attn_forward_gqa(q.float(), k[:, :, :2].float(), k[:, :, :2].float())
