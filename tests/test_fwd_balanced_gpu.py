"""The balanced causal forward (fa_fwd_ws on square causal grids of at least 32
query tiles per head and at most half a tile per compute unit, one from 48
tiles per head, 1.75 from 64) against the float64 oracle and against the
plain schedule.

The schedule pairs light causal query tiles with heavy ones, cuts each
pair in three work items (the heavy tile's two key halves and the light
tile) and merges the heavy tile's halves with fa_fwd_combine_kernel
(fa_fwd.hpp, fa_fwd_bal_item).  Cases cover an even and an odd number of
tiles per head (the odd middle tile) with a ragged last tile, every head
dimension, batches, grouped heads, bf16, a scale above the pre-scaled
mode's bound and a negative one.  Tolerance: max-abs 1e-2 on
O and LSE against the oracle for fp16 outputs, 4e-2 for bf16 (the
suite's bars); the two schedules differ in the rounding of the merge
only: at most four output ulps apart.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

TOL = 1e-2
BF16_TOL = 4e-2

CASES = [
    # B, S, H, Hk, D, dtype, sm_scale
    (1, 4096, 4, 4, 128, torch.float16, None),     # 64 tiles x 4 heads: one per CU
    (1, 4096, 6, 3, 128, torch.float16, None),     # 1.5 tiles per CU, grouped heads
    (1, 4096, 7, 7, 64, torch.bfloat16, None),     # 1.75 tiles per CU
    (1, 3100, 3, 3, 64, torch.float16, None),      # 49 tiles: odd, ragged, under 64
    (2, 2048, 2, 1, 128, torch.float16, None),     # 32 tiles, half a tile per CU, grouped
    (1, 4100, 2, 2, 64, torch.float16, None),      # 65 tiles: odd middle tile, ragged
    (2, 4096, 1, 1, 32, torch.float16, None),      # D = 32, two batches
    (1, 4096, 4, 2, 128, torch.float16, None),     # grouped heads
    (1, 4096, 2, 2, 64, torch.bfloat16, None),     # bf16
    (1, 4096, 1, 1, 64, torch.float16, 2.0),       # c > 1: scale applied in the softmax
    (1, 4096, 1, 1, 64, torch.float16, -0.125),    # negative scale
]


def _ids(c):
    B, S, H, Hk, D, dt, sc = c
    return f"B{B}S{S}H{H}/{Hk}D{D}{'bf16' if dt == torch.bfloat16 else 'f16'}s{sc}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_balanced_forward(case):
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import _DTYPES, kernel_strides
    B, S, H, Hk, D, dt, sm_scale = case
    print(f"[case] balanced forward {_ids(case)}", flush=True)
    lib = _capi.load()
    nbytes = lib.fa_fwd_workspace_bytes(B, S, S, H, Hk, D, 1)
    assert nbytes > 0, "the balanced schedule should apply to this grid"
    g = torch.Generator(device="cpu").manual_seed(3)
    q = torch.randn((B, S, H, D), generator=g).to(dt)
    k = torch.randn((B, S, Hk, D), generator=g).to(dt)
    v = torch.randn((B, S, Hk, D), generator=g).to(dt)
    sc = D ** -0.5 if sm_scale is None else sm_scale
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    st_q, st_k = kernel_strides(qd), kernel_strides(kd)
    stream = torch.cuda.current_stream().cuda_stream

    def run(ws):
        out = torch.empty_like(qd)
        lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
        if ws is None:
            rc = lib.fa_fwd_gqa(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                lse.data_ptr(), B, S, S, H, Hk, D, st_q, st_k, st_k, st_q,
                                sc, 1, _DTYPES[dt], stream)
        else:
            rc = lib.fa_fwd_ws(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                               lse.data_ptr(), ws.data_ptr(), ws.numel(), B, S, S, H, Hk, D,
                               st_q, st_k, st_k, st_q, sc, 1, _DTYPES[dt], stream)
        _capi.check(rc, "forward")
        return out, lse

    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ws.fill_(0xFF)                    # no reliance on a zeroed workspace
    o_b, l_b = run(ws)
    o_b2, l_b2 = run(ws)              # reproducible
    o_p, l_p = run(None)
    torch.cuda.synchronize()
    assert torch.equal(o_b, o_b2) and torch.equal(l_b, l_b2)
    o_ref, l_ref = orc.attention_fwd_gqa(q.float(), k.float(), v.float(), True, sc)
    err_o = float(np.abs(o_b.double().cpu().numpy() - o_ref).max())
    err_l = float(np.abs(l_b.double().cpu().numpy() - l_ref).max())
    print(f"[case] max-abs O {err_o:.3e} LSE {err_l:.3e}", flush=True)
    tol = BF16_TOL if dt == torch.bfloat16 else TOL
    assert err_o < tol and err_l < tol
    # against the plain schedule: the merge's rounding only -- within four
    # ulps of the output type (spacing <= 2^-10 |x| in fp16, 2^-7 |x| in
    # bf16, taken at |x| >= 1)
    eps = 2.0 ** -7 if dt == torch.bfloat16 else 2.0 ** -10
    bound = 4 * eps * o_p.float().abs().clamp_min(1.0)
    assert bool(((o_b.float() - o_p.float()).abs() <= bound).all())
    # LSE = m + log(l), l a sum of probabilities rounded to the input type
    # against each half's own max: a dominant probability's rounding moves
    # l by up to 2^-11 (fp16) or 2^-8 (bf16) relative, LSE by about as much
    assert (l_b - l_p).abs().max().item() < (8e-3 if dt == torch.bfloat16 else 1e-3)


def test_balanced_forward_through_wrappers():
    """flash_attn_forward and flash_attn (autograd, C++ node) take the
    balanced schedule for a shape it applies to; the backward then runs on
    its O and LSE, within the suite's tolerance of the oracle."""
    from flash_attn_volta import _capi, flash_attn, flash_attn_forward
    B, S, H, D = 1, 4096, 2, 128
    assert _capi.load().fa_fwd_workspace_bytes(B, S, S, H, H, D, 1) > 0
    print("[case] balanced forward through the wrappers", flush=True)
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=4, scale=0.5)
    qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
    o, lse = flash_attn_forward(qd, kd, vd, causal=True, return_softmax_lse=True)
    o_ref, l_ref = orc.attention_fwd(q, k, v, True)
    assert float(np.abs(o.double().cpu().numpy() - o_ref).max()) < TOL
    assert float(np.abs(lse.double().cpu().numpy() - l_ref).max()) < TOL
    qg, kg, vg = (t.clone().requires_grad_() for t in (qd, kd, vd))
    out = flash_attn(qg, kg, vg, causal=True)
    out.backward(dod)
    dq_ref, dk_ref, dv_ref, _ = orc.attention_bwd(do, q, k, v, True, o=o_ref)
    for got, ref in ((out, o_ref), (qg.grad, dq_ref), (kg.grad, dk_ref), (vg.grad, dv_ref)):
        assert float(np.abs(got.detach().double().cpu().numpy() - ref).max()) < TOL
