"""Split-KV forward (decode against a long cache) on the GPU: fa_fwd_splitkv
through flash_attn_forward_gqa / flash_attn_gqa, against the float64 oracle
(attention_fwd_gqa / attention_bwd_gqa) on identical seeded 16-bit inputs,
and against the unsplit kernel (fa_fwd_gqa).

Tolerance: max-abs 1e-2 on O, LSE and gradients for fp16, 4e-2 for bf16, as
for every other forward; the split and unsplit kernels agree to 2e-3 (fp16)
/ 1.6e-2 (bf16) on O and 1e-4 / 1e-3 on LSE (they differ in the order of
their fp32 sums, in one rounding of O, and in the maxima the 16-bit
probabilities are rounded against).

Cases: single-token decode with GQA groups of 1..8 heads, a query block of
several positions (speculative decode / small chunks) whose rows see
different key counts (so some key ranges are empty for some rows), ragged
key lengths, the largest packed tile (64 rows), D = 32/64/128, causal and
not, fp16 and bf16; the backward through the split forward's LSE.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import TOL, default_scale, max_abs
from oracle import attention as orc

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16

# (B, Sq, Sk, H, Hk, D, causal, dtype)
CASES = [
    (1, 1, 4096, 32, 8, 128, True, F16),
    (2, 1, 1000, 8, 1, 64, True, F16),
    (1, 4, 2048, 16, 4, 128, True, BF16),
    (1, 8, 8192, 64, 8, 128, True, F16),
    (3, 1, 777, 4, 4, 32, False, F16),
    (1, 2, 300, 8, 8, 64, True, F16),
    (1, 16, 5000, 8, 2, 64, True, F16),
    (2, 3, 3333, 12, 3, 128, False, BF16),
]


def _ids(c):
    B, Sq, Sk, H, Hk, D, causal, dt = c
    return f"B{B}Sq{Sq}Sk{Sk}H{H}Hk{Hk}D{D}{'c' if causal else 'n'}-{'bf16' if dt == BF16 else 'f16'}"


def _splits(B, Sq, Sk, H, Hk, D):
    from flash_attn_volta import _capi
    return _capi.load().fa_fwd_splitkv_workspace_bytes(B, Sq, Sk, H, Hk, D)


def _unsplit(q, k, v, causal):
    """The regular kernel through the C ABI (fa_fwd_gqa), for comparison."""
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import _DTYPES, kernel_strides
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
    rc = _capi.load().fa_fwd_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                 lse.data_ptr(), B, Sq, Sk, H, Hk, D, kernel_strides(q),
                                 kernel_strides(k), kernel_strides(v), kernel_strides(o),
                                 default_scale(D, None), int(causal), _DTYPES[q.dtype],
                                 torch.cuda.current_stream().cuda_stream)
    _capi.check(rc, "fa_fwd_gqa")
    return o, lse


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_splitkv_forward_matches_oracle_and_unsplit(case):
    from flash_attn_volta import flash_attn_forward_gqa
    B, Sq, Sk, H, Hk, D, causal, dtype = case
    print(f"[decode] case {_ids(case)}", flush=True)
    assert _splits(B, Sq, Sk, H, Hk, D) > 0, "the split path must be taken for this case"
    q, k, v, _ = orc.make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=31, dtype=dtype)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    o, lse = flash_attn_forward_gqa(qd, kd, vd, causal=causal, return_softmax_lse=True)
    o2, lse2 = _unsplit(qd, kd, vd, causal)
    torch.cuda.synchronize()
    ro, rlse = orc.attention_fwd_gqa(q, k, v, causal, default_scale(D, None))
    tol = TOL if dtype == F16 else 4e-2
    eo, el = max_abs(o, ro), max_abs(lse, rlse)
    d_o, d_l = max_abs(o, o2), max_abs(lse, lse2)
    print(f"[decode] vs oracle: o {eo:.3e} lse {el:.3e}; vs unsplit: o {d_o:.3e} lse {d_l:.3e}",
          flush=True)
    assert eo <= tol and el <= tol
    assert d_o <= (2e-3 if dtype == F16 else 1.6e-2) and d_l <= (1e-4 if dtype == F16 else 1e-3)


@pytest.mark.parametrize("case", [CASES[0], CASES[6], CASES[2]], ids=[_ids(c) for c in (CASES[0], CASES[6], CASES[2])])
def test_backward_through_split_forward(case):
    from flash_attn_volta import flash_attn_gqa
    B, Sq, Sk, H, Hk, D, causal, dtype = case
    q, k, v, do = orc.make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=32, dtype=dtype)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    out = flash_attn_gqa(qd, kd, vd, causal=causal)
    out.backward(do.cuda())
    torch.cuda.synchronize()
    sc = default_scale(D, None)
    ro, _ = orc.attention_fwd_gqa(q, k, v, causal, sc)
    rdq, rdk, rdv, _ = orc.attention_bwd_gqa(do, q, k, v, causal, sc)
    tol = TOL if dtype == F16 else 4e-2
    errs = [max_abs(out, ro), max_abs(qd.grad, rdq), max_abs(kd.grad, rdk), max_abs(vd.grad, rdv)]
    print(f"[decode] bwd {_ids(case)} o/dq/dk/dv " + " ".join(f"{e:.3e}" for e in errs), flush=True)
    assert max(errs) <= tol


def test_split_path_is_deterministic():
    from flash_attn_volta import flash_attn_forward_gqa
    q, k, v, _ = orc.make_inputs_gqa(1, 1, 4096, 32, 8, 128, seed=33)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    a = flash_attn_forward_gqa(qd, kd, vd, causal=True, return_softmax_lse=True)
    b = flash_attn_forward_gqa(qd, kd, vd, causal=True, return_softmax_lse=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
