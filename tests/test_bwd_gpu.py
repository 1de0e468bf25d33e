"""Backward parity on the GPU: flash_attn (autograd) and flash_attn_backward
(HIP kernels via the C ABI) against the float64 CPU oracle.

Mirrors the reference's backward suite (tests/test_backward.py): grads vs
float64 SDPA+autograd (:145-179; the reference allowed 2e-2, this build
holds 1e-2 as BASELINE requires), the finite-difference gradcheck on a tiny
causal shape (:182-277) and the bitwise causal no-leak check (:280-320).
Adds every BASELINE config at full size, ragged lengths, signed scales,
the delta pre-pass and bitwise run-to-run determinism.
"""
from __future__ import annotations

import functools
import math

import numpy as np
import pytest
import torch

from helpers import CONFIGS, TOL, default_scale, max_abs, report
from oracle import attention as orc

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=2)
def _oracle(B, S, H, D, causal, sm_scale, in_scale, seed):
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=seed, scale=in_scale)
    sc = default_scale(D, sm_scale)
    o, lse = orc.attention_fwd(q, k, v, causal, sc)
    dq, dk, dv, delta = orc.attention_bwd(do, q, k, v, causal, sc, o=o)
    return (q, k, v, do), (o, lse, dq, dk, dv, delta)


def _autograd(q, k, v, do, causal, sm_scale):
    from flash_attn_volta import flash_attn
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    out = flash_attn(qg, kg, vg, causal=causal, sm_scale=sm_scale)
    out.backward(do.cuda())
    torch.cuda.synchronize()
    return out.detach(), qg.grad, kg.grad, vg.grad


BWD_CONFIGS = [c for c in CONFIGS if c[0] != "C1"]   # C1 is forward-only


@pytest.mark.parametrize("cfg", BWD_CONFIGS, ids=[c[0] for c in BWD_CONFIGS])
def test_backward_configs(cfg):
    name, B, S, H, D, causal, sm_scale, in_scale = cfg
    print(f"[case] bwd {name} B={B} S={S} H={H} D={D} causal={causal}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv, _) = _oracle(B, S, H, D, causal, sm_scale, in_scale, 0)
    out, gq, gk, gv = _autograd(q, k, v, do, causal, sm_scale)
    errs = dict(out=max_abs(out, o), dq=max_abs(gq, dq), dk=max_abs(gk, dk), dv=max_abs(gv, dv))
    report(f"bwd {name}", **errs)
    for key, e in errs.items():
        assert e < TOL, f"{name} {key} max-abs {e:.3e} >= {TOL}"


# The reference's backward shapes (tests/test_backward.py:122-127).
@pytest.mark.parametrize("shape", [(2, 1024, 8, 64), (1, 2048, 16, 128), (4, 512, 4, 32), (1, 64, 2, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_reference_shapes(shape, causal):
    B, S, H, D = shape
    print(f"[case] bwd ref-shape {shape} causal={causal}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv, _) = _oracle(B, S, H, D, causal, None, 1.0, 1)
    out, gq, gk, gv = _autograd(q, k, v, do, causal, None)
    errs = dict(out=max_abs(out, o), dq=max_abs(gq, dq), dk=max_abs(gk, dk), dv=max_abs(gv, dv))
    report(f"bwd {shape} c={int(causal)}", **errs)
    assert max(errs.values()) < TOL


@pytest.mark.parametrize("S", [1, 17, 33, 65, 100, 255, 513])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_ragged(S, D, causal):
    B, H = 2, 2
    print(f"[case] bwd ragged S={S} D={D} causal={causal}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv, _) = _oracle(B, S, H, D, causal, None, 1.0, 2)
    out, gq, gk, gv = _autograd(q, k, v, do, causal, None)
    assert max(max_abs(gq, dq), max_abs(gk, dk), max_abs(gv, dv), max_abs(out, o)) < TOL


# 1.0 and -1.2 exceed ln 2: the dK/dV kernel then applies the part of the
# scale that K's pre-multiplication leaves out (cr != 1) to the scores.
# Their inputs are scaled by 0.35 so the scores keep the spread of the
# default scale (std ~1; at std ~8 the fp16 rounding of dS alone moves dQ by
# more than the 1e-2 bound).
@pytest.mark.parametrize("sm_scale", [-0.1, 0.0, 0.3, 1.0, -1.2])
def test_backward_signed_and_zero_scale(sm_scale):
    B, S, H, D = 1, 200, 2, 64
    in_scale = 0.35 if abs(sm_scale) > 0.7 else 1.0
    print(f"[case] bwd scale={sm_scale} inputs x{in_scale}", flush=True)
    (q, k, v, do), (o, lse, dq, dk, dv, _) = _oracle(B, S, H, D, True, sm_scale, in_scale, 4)
    out, gq, gk, gv = _autograd(q, k, v, do, True, sm_scale)
    assert max(max_abs(gq, dq), max_abs(gk, dk), max_abs(gv, dv)) < TOL


def test_backward_direct_call_matches_autograd():
    from flash_attn_volta import flash_attn_backward, flash_attn_forward
    B, S, H, D = 2, 300, 3, 64
    q, k, v, do = (t.cuda() for t in orc.make_inputs(B, S, H, D, seed=5))
    out, lse = flash_attn_forward(q, k, v, causal=True, return_softmax_lse=True)
    dq, dk, dv = flash_attn_backward(do, q, k, v, out, lse, causal=True)
    _, gq, gk, gv = _autograd(q.cpu(), k.cpu(), v.cpu(), do.cpu(), True, None)
    assert torch.equal(dq, gq) and torch.equal(dk, gk) and torch.equal(dv, gv)


def test_delta_preprocess_matches_oracle():
    from flash_attn_volta.backward import bwd_preprocess
    for D in (32, 64, 128):
        q, k, v, do = orc.make_inputs(2, 333, 3, D, seed=6)
        delta = bwd_preprocess(q.cuda(), do.cuda())   # any two fp16 tensors
        ref = (q.double() * do.double()).sum(-1).permute(0, 2, 1)
        assert max_abs(delta, ref) < 1e-3


def test_backward_finite_difference_subset():
    """Reference tests/test_backward.py:182-277: central differences (here in
    float64 through the oracle forward) on 8 random coordinates of each of
    Q, K, V at (1, 16, 2, 32) causal, vs the kernel's analytic grads;
    pass if abs < 5e-3 or rel < 5e-2 per the reference's budget."""
    B, S, H, D = 1, 16, 2, 32
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=0)
    scale = 1.0 / math.sqrt(D)
    _, gq, gk, gv = _autograd(q, k, v, do, True, scale)
    q64, k64, v64, do64 = (t.double().numpy() for t in (q, k, v, do))

    def loss(qq, kk, vv):
        return float((orc.attention_fwd(qq, kk, vv, True, scale)[0] * do64).sum())

    rng = np.random.default_rng(42)
    h = 1e-4
    worst_abs = worst_rel = 0.0
    for which, grad in enumerate((gq, gk, gv)):
        g = grad.double().cpu().numpy()
        for flat in rng.choice(q64.size, size=8, replace=False):
            idx = np.unravel_index(flat, q64.shape)
            args_p = [q64.copy(), k64.copy(), v64.copy()]
            args_m = [q64.copy(), k64.copy(), v64.copy()]
            args_p[which][idx] += h
            args_m[which][idx] -= h
            fd = (loss(*args_p) - loss(*args_m)) / (2 * h)
            err = abs(fd - g[idx])
            worst_abs = max(worst_abs, err)
            worst_rel = max(worst_rel, err / max(abs(fd), 1e-3))
    print(f"[fd] worst_abs={worst_abs:.3e} worst_rel={worst_rel:.3e}", flush=True)
    assert worst_abs < 5e-3 or worst_rel < 5e-2


def test_backward_causal_no_leak():
    """Reference tests/test_backward.py:280-320: perturbing K, V at j >= N/2
    leaves dQ of rows < N/2 bit-identical and changes later rows."""
    B, N, H, D = 1, 64, 2, 64
    q, k, v, do = orc.make_inputs(B, N, H, D, seed=0)
    _, dq_a, _, _ = _autograd(q, k, v, do, True, None)
    gen = torch.Generator("cpu").manual_seed(3)
    k_p, v_p = k.clone(), v.clone()
    j = N // 2
    k_p[:, j:] += (torch.randn(k_p[:, j:].shape, generator=gen) * 0.5).half()
    v_p[:, j:] += (torch.randn(v_p[:, j:].shape, generator=gen) * 0.5).half()
    _, dq_b, _, _ = _autograd(q, k_p, v_p, do, True, None)
    leak = (dq_a[:, :j] - dq_b[:, :j]).abs().max().item()
    late = (dq_a[:, j:] - dq_b[:, j:]).abs().max().item()
    assert leak == 0.0, f"causal leak {leak:.3e}"
    assert late > 1e-3


def test_backward_is_deterministic():
    B, S, H, D = 1, 1024, 4, 128
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=7)
    a = _autograd(q, k, v, do, True, None)
    b = _autograd(q, k, v, do, True, None)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("D", [64, 128])
def test_backward_tiny_upstream_gradient(D):
    """dO ~ 1e-6 (fp16 subnormals, as deep in an fp16 network trained without
    loss scaling): dS then lies far below the fp16 normal range, and rounding
    it to fp16 unscaled flushes ~all of it to zero.  The kernels' per-row
    power-of-two dS scaling must keep the gradients as good as an fp32 eager
    attention whose gradients are likewise returned in fp16."""
    B, S, H = 1, 1024, 4
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=9)
    do = (do.float() * 2.0 ** -20).half()
    _, gq, gk, gv = _autograd(q, k, v, do, True, None)
    qh, kh, vh = (t.cuda().requires_grad_() for t in (q, k, v))
    q32, k32, v32 = (t.float().permute(0, 2, 1, 3).contiguous() for t in (qh, kh, vh))
    s = torch.matmul(q32, k32.transpose(-1, -2).contiguous()) / math.sqrt(D)
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device="cuda"), 1), float("-inf"))
    o = torch.matmul(torch.softmax(s, -1), v32).permute(0, 2, 1, 3).half()
    o.backward(do.cuda())
    for name, ours, ref in (("dq", gq, qh.grad), ("dk", gk, kh.grad), ("dv", gv, vh.grad)):
        a, b = ours.double().flatten(), ref.double().flatten()
        cos = float(a @ b / (a.norm() * b.norm()))
        zeros = (ours == 0).float().mean().item()
        print(f"[tiny-dO] D={D} {name}: cos vs fp32-eager {cos:.6f}, zero fraction {zeros:.4f}", flush=True)
        assert cos >= 0.9999, f"{name} cos {cos}"
        assert zeros <= (ref == 0).float().mean().item() + 1e-3


# Large enough grids to run the unsplit backward kernels (the launcher splits
# rows across waves only for grids under 2 / 4 (causal) workgroups per CU).
@pytest.mark.parametrize("shape,causal,sm_scale", [((4, 1000, 32, 64), False, None),
                                                   ((8, 600, 32, 32), True, None),
                                                   ((2, 1100, 64, 128), False, None),
                                                   ((2, 1100, 32, 128), True, None),
                                                   ((1, 600, 64, 128), False, 1.0)])
def test_backward_large_grid_variant(shape, causal, sm_scale):
    B, S, H, D = shape
    print(f"[case] bwd large-grid {shape} causal={causal} scale={sm_scale}", flush=True)
    in_scale = 0.35 if sm_scale is not None and abs(sm_scale) > 0.7 else 1.0
    (q, k, v, do), (o, lse, dq, dk, dv, _) = _oracle(B, S, H, D, causal, sm_scale, in_scale, 11)
    out, gq, gk, gv = _autograd(q, k, v, do, causal, sm_scale)
    assert max(max_abs(gq, dq), max_abs(gk, dk), max_abs(gv, dv), max_abs(out, o)) < TOL


def test_backward_upstream_rows_of_very_different_magnitude():
    """dO rows scaled by 2^-20 .. 2^-6 (one power per query) and V entries up
    to ~2000, sized so every true gradient fits fp16: the dQ kernel's fixed
    per-query scale (from the query's own dO row) puts each row's largest
    |dO| in [2^-4, 2^-3), so its scaled dS reaches up to
    2^-2 * D * max|V| ~ 32000, near but inside fp16; tiny rows must keep
    their precision.  The dK/dV kernel's running scale must handle the mix.
    dQ rows are checked against their own magnitude (max-abs <= 1e-2 of the
    row's largest value, plus two fp16 subnormal steps); dK and dV against
    theirs."""
    B, S, H, D = 1, 512, 2, 64
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=41)
    g = torch.Generator("cpu").manual_seed(42)
    v = (v.float() * 512.0).half()
    e = torch.randint(-20, -5, (1, S, 1, 1), generator=g).float()
    do = (do.float() * torch.exp2(e)).half()
    sc = default_scale(D, None)
    o, _ = orc.attention_fwd(q, k, v, True, sc)
    rdq, rdk, rdv, _ = orc.attention_bwd(do, q, k, v, True, sc, o=o)
    _, gq, gk, gv = _autograd(q, k, v, do, True, None)
    gq = gq.double().cpu().numpy()
    row_ref = np.abs(rdq).max(axis=-1, keepdims=True)
    row_err = np.abs(gq - rdq).max(axis=-1, keepdims=True)
    worst = float(np.max(row_err / (1e-2 * row_ref + 2.0 ** -23)))
    ek = max_abs(gk, rdk) / float(np.abs(rdk).max())
    ev = max_abs(gv, rdv) / float(np.abs(rdv).max())
    print(f"[mixed-dO] dq worst row err/bound {worst:.3f}; dk rel {ek:.3e}; dv rel {ev:.3e}",
          flush=True)
    assert np.all(np.isfinite(gq)) and worst <= 1.0
    assert ek <= 1e-2 and ev <= 1e-2


def _bwd_capi(do, q, k, v, o, lse, causal, ws_bytes, fill):
    """fa_bwd_gqa through the C ABI with a workspace of `ws_bytes` bytes, every
    byte set to `fill` first (stale split counters and partials)."""
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.full((ws_bytes,), fill, dtype=torch.uint8, device="cuda")
    st = tuple(kernel_strides(t) for t in (do, q, k, v, o, dq, dk, dv))
    dtype = _capi.FA_DTYPE_F16 if q.dtype == torch.float16 else _capi.FA_DTYPE_BF16
    rc = lib.fa_bwd_gqa(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                        lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                        ws.data_ptr(), ws_bytes, B, Sq, Sk, H, Hk, D, *st,
                        1.0 / math.sqrt(D), int(causal), dtype,
                        torch.cuda.current_stream().cuda_stream)
    _capi.check(rc, "fa_bwd_gqa")
    torch.cuda.synchronize()
    return dq, dk, dv


# Causal D = 64 / 128 problems whose key blocks fit one round of resident
# workgroups: with the workspace fa_bwd_gqa_workspace_bytes sizes, the
# longest key blocks are swept by two workgroups whose fp32 partials the
# second to finish adds; likewise the dQ kernel's longest query blocks,
# whose halves the dK/dV kernel adds (every case splits dQ, which is when
# the key split runs -- without it the fused launch runs unsplit, as it
# does on sweeps under 64 key tiles; the second, third and fifth have a
# ragged last query block among their split ones).
@pytest.mark.parametrize("B,Sq,Sk,H,Hk,D,dtype", [
    (1, 4096, 4096, 4, 4, 128, torch.float16),
    (1, 3000, 4200, 4, 2, 128, torch.float16),    # grouped heads, offset 1200, ragged split block
    (1, 4100, 4100, 2, 2, 128, torch.bfloat16),   # ragged last key block (unsplit)
    (1, 4096, 4096, 4, 4, 64, torch.float16),
    (1, 3000, 4096, 8, 2, 64, torch.bfloat16),    # grouped heads, offset 1096
    (2, 4096, 4096, 2, 2, 128, torch.float16),     # batch 2: slots and dQ rows per (b, h)
    (2, 4096, 4096, 2, 1, 64, torch.float16),      # batch 2, grouped heads
])
def test_backward_causal_key_block_split(B, Sq, Sk, H, Hk, D, dtype):
    from flash_attn_volta import _capi, flash_attn_forward_gqa
    print(f"[case] bwd key-block split B={B} Sq={Sq} Sk={Sk} H={H} Hk={Hk} D={D} {dtype}", flush=True)
    lib = _capi.load()
    full = lib.fa_bwd_gqa_workspace_bytes(B, Sq, Sk, H, Hk, D, 1)
    minimum = lib.fa_bwd_workspace_bytes(B, Sq, H, D)
    assert full > minimum, "the split must apply to this shape"
    q, k, v, do = orc.make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=13, dtype=dtype)
    sc = default_scale(D, None)
    o_ref, _ = orc.attention_fwd_gqa(q, k, v, True, sc)
    dq_ref, dk_ref, dv_ref, _ = orc.attention_bwd_gqa(do, q, k, v, True, sc, o=o_ref)
    qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
    o, lse = flash_attn_forward_gqa(qd, kd, vd, causal=True, return_softmax_lse=True)
    unsplit = _bwd_capi(dod, qd, kd, vd, o, lse, True, minimum, 0)
    split = _bwd_capi(dod, qd, kd, vd, o, lse, True, full, 0xFF)
    again = _bwd_capi(dod, qd, kd, vd, o, lse, True, full, 0x00)
    tol = TOL if dtype == torch.float16 else 4e-2
    errs = dict(dq=max_abs(split[0], dq_ref), dk=max_abs(split[1], dk_ref),
                dv=max_abs(split[2], dv_ref))
    report(f"bwd split {B},{Sq},{Sk},{H},{Hk}", **errs)
    for key, e in errs.items():
        assert e < tol, f"{key} max-abs {e:.3e} >= {tol}"
    # split and unsplit differ by rounding only
    for a, b in zip(split, unsplit):
        assert max_abs(a, b.float()) < tol / 4
    # bit-reproducible whatever the workspace held before
    for a, b in zip(split, again):
        assert torch.equal(a, b)


def _bwd_three_launches(do, q, k, v, o, lse, causal, sm_scale):
    """The three separate entry points fa_bwd_preprocess, fa_bwd_dq and
    fa_bwd_dkdv (the reference's three backward launches), fp16."""
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    B, S, H, D = q.shape
    stream = torch.cuda.current_stream().cuda_stream
    delta = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
    rowmax = torch.empty(lib.fa_bwd_rowmax_bytes(B, S, H) // 4, dtype=torch.float32, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    st = {n: kernel_strides(t) for n, t in dict(do=do, q=q, k=k, v=v, o=o, dq=dq, dk=dk,
                                                   dv=dv).items()}
    _capi.check(lib.fa_bwd_preprocess(o.data_ptr(), do.data_ptr(), delta.data_ptr(),
                                      rowmax.data_ptr(), B, S, H, D, st["o"], st["do"], stream),
                "fa_bwd_preprocess")
    _capi.check(lib.fa_bwd_dq(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                              lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), B, S, H, D,
                              st["do"], st["q"], st["k"], st["v"], st["dq"], sm_scale,
                              int(causal), stream), "fa_bwd_dq")
    _capi.check(lib.fa_bwd_dkdv(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                lse.data_ptr(), delta.data_ptr(), rowmax.data_ptr(),
                                dk.data_ptr(), dv.data_ptr(),
                                B, S, H, D, st["do"], st["q"], st["k"], st["v"], st["dk"],
                                st["dv"], sm_scale, int(causal), stream), "fa_bwd_dkdv")
    torch.cuda.synchronize()
    # fa_bwd_blocks: both gradient launches of fa_bwd, given the same delta
    # and row-group maxima
    bq, bk, bv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    _capi.check(lib.fa_bwd_blocks(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  lse.data_ptr(), delta.data_ptr(), rowmax.data_ptr(),
                                  bq.data_ptr(), bk.data_ptr(),
                                  bv.data_ptr(), B, S, H, D, st["do"], st["q"], st["k"], st["v"],
                                  st["dq"], st["dk"], st["dv"], sm_scale, int(causal), stream),
                "fa_bwd_blocks")
    torch.cuda.synchronize()
    return (dq, dk, dv), (bq, bk, bv)


# The causal backward runs as the pre-pass and one fused launch (every
# dK/dV block, then every dQ block, in one grid: four-wave blocks at
# D = 32 / 64, eight-wave ones at D = 128); the three separate entry points
# run the same block code in three launches, so the gradients must be
# bit-identical; so must fa_bwd_blocks (the fused launch alone, given
# delta).  Shapes: both layout pairs the launcher picks for H = Hk at
# D = 64 (dK/dV query-split with dQ key-split on grids under a round, both
# unsplit above), a ragged length, a scale above ln 2 (the dQ block's
# unscaled mode), and D = 128 grids on which flash_attn_backward's
# workspace enables no key-block split (a split sums two fp32 partials, a
# different rounding; its own test is test_backward_causal_key_block_split).
@pytest.mark.parametrize("B,S,H,D,sm_scale,in_scale", [
    (1, 4096, 16, 64, None, 0.5),
    (4, 2048, 16, 64, None, 1.0),
    (1, 2048, 8, 64, None, 1.0),       # half a round: fused in place of the dQ split
    (2, 1000, 8, 64, 1.0, 0.35),
    (4, 512, 4, 32, None, 1.0),
    (8, 1024, 32, 32, None, 1.0),
    (1, 4096, 16, 128, None, 0.5),
    (2, 1100, 32, 128, None, 1.0),
    (1, 2048, 16, 128, 1.0, 0.35),
    (2, 2048, 32, 128, None, 1.0),     # four rounds of D = 128 dK/dV blocks, still fused
])
def test_backward_fused_launch_matches_three_launches(B, S, H, D, sm_scale, in_scale):
    from flash_attn_volta import flash_attn_backward, flash_attn_forward
    print(f"[case] bwd fused vs three launches B={B} S={S} H={H} D={D} scale={sm_scale}",
          flush=True)
    q, k, v, do = (t.cuda() for t in orc.make_inputs(B, S, H, D, seed=21, scale=in_scale))
    sc = default_scale(D, sm_scale)
    o, lse = flash_attn_forward(q, k, v, causal=True, sm_scale=sc, return_softmax_lse=True)
    fused = flash_attn_backward(do, q, k, v, o, lse, causal=True, sm_scale=sc)
    three, blocks = _bwd_three_launches(do, q, k, v, o, lse, True, sc)
    for name, a, b, c in zip(("dq", "dk", "dv"), fused, three, blocks):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, b), f"{name} differs (max-abs {max_abs(a, b.float()):.3e})"
        assert torch.equal(a, c), f"fa_bwd_blocks {name} differs"


# fa_bwd's dK/dV blocks read row-group maxima -- max |dO| and max |delta|
# over every 32 query rows of each (b, h), which bound |dS| and so fix each
# query tile's dS scale -- written by the dQ kernel on the unfused shapes
# (the pre-pass folded into it) and by the pre-pass on the fused causal
# D <= 64 ones.  Both must equal the maxima of dO and of the delta the
# same call wrote (bitwise: a max is exact; groups past S hold nothing),
# fa_bwd_preprocess must write the same delta and maxima, and the three
# separate launches, which read the pre-pass's maxima, must reproduce
# fa_bwd bit for bit.  dO rows span 2^-6 .. 2^2, so a group boundary off
# by a row changes a maximum.
@pytest.mark.parametrize("B,S,H,D,causal", [
    (1, 1000, 4, 128, True),    # unfused causal, ragged last group
    (2, 777, 3, 64, False),     # unfused non-causal
    (1, 1024, 8, 128, False),
    (2, 300, 2, 32, False),
    (2, 1000, 8, 64, True),     # fused: the pre-pass writes them
])
def test_backward_row_maxima(B, S, H, D, causal):
    from flash_attn_volta import _capi, flash_attn_forward
    from flash_attn_volta.forward import kernel_strides
    print(f"[case] bwd row maxima B={B} S={S} H={H} D={D} causal={causal}", flush=True)
    lib = _capi.load()
    q, k, v, do = (t.cuda() for t in orc.make_inputs(B, S, H, D, seed=31))
    g = torch.Generator("cpu").manual_seed(32)
    e = torch.randint(-6, 3, (1, S, 1, 1), generator=g).float().cuda()
    do = (do.float() * torch.exp2(e)).half()
    sc = default_scale(D, None)
    o, lse = flash_attn_forward(q, k, v, causal=causal, sm_scale=sc, return_softmax_lse=True)
    G = (S + 31) // 32
    r_bytes = lib.fa_bwd_rowmax_bytes(B, S, H)
    ws_bytes = lib.fa_bwd_workspace_bytes(B, S, H, D)
    d_bytes = ws_bytes - r_bytes
    assert r_bytes >= B * H * G * 8 and d_bytes >= B * H * S * 4
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    st = tuple(kernel_strides(t) for t in (do, q, k, v, o, dq, dk, dv))
    stream = torch.cuda.current_stream().cuda_stream
    _capi.check(lib.fa_bwd(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                           lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                           ws.data_ptr(), ws_bytes, B, S, H, D, *st, sc, int(causal), stream),
                "fa_bwd")
    torch.cuda.synchronize()
    delta = ws[:d_bytes].view(torch.float32)[:B * H * S].view(B, H, S)
    rmax = ws[d_bytes:].view(torch.float32)[:B * H * G * 2].view(B, H, G, 2)
    pad = G * 32 - S
    mdo = do.float().abs().amax(-1).permute(0, 2, 1)                # (B, H, S)
    mdo = torch.nn.functional.pad(mdo, (0, pad)).view(B, H, G, 32).amax(-1)
    mdl = torch.nn.functional.pad(delta.abs(), (0, pad)).view(B, H, G, 32).amax(-1)
    assert torch.equal(rmax[..., 0], mdo), "max |dO| per group"
    assert torch.equal(rmax[..., 1], mdl), "max |delta| per group"
    ref_delta = (o.double() * do.double()).sum(-1).permute(0, 2, 1)
    assert max_abs(delta, ref_delta) < 1e-3
    # the pre-pass's delta and maxima, and the three launches
    d2 = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
    r2 = torch.full((r_bytes // 4,), float("nan"), dtype=torch.float32, device="cuda")
    _capi.check(lib.fa_bwd_preprocess(o.data_ptr(), do.data_ptr(), d2.data_ptr(), r2.data_ptr(),
                                      B, S, H, D, st[4], st[0], stream), "fa_bwd_preprocess")
    torch.cuda.synchronize()
    assert torch.equal(d2, delta)
    assert torch.equal(r2[:B * H * G * 2].view(B, H, G, 2), rmax)
    three, blocks = _bwd_three_launches(do, q, k, v, o, lse, causal, sc)
    for name, a, b, c in zip(("dq", "dk", "dv"), (dq, dk, dv), three, blocks):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, b), f"{name} differs (max-abs {max_abs(a, b.float()):.3e})"
        assert torch.equal(a, c), f"fa_bwd_blocks {name} differs"


# The two mixed layout pairs, which need H != Hk or Sq != Sk (so the three
# square entry points cannot run them): dK/dV query-split beside unsplit dQ
# (many query heads per key/value head), and unsplit dK/dV beside the
# key-split dQ (a short query block against a long key range, bottom-right
# causal); against the float64 oracle, fp16 and bf16.
@pytest.mark.parametrize("B,Sq,Sk,H,Hk,D,dtype", [
    (32, 128, 128, 32, 4, 32, torch.float16),
    (32, 128, 128, 32, 4, 32, torch.bfloat16),
    (4, 128, 1024, 32, 32, 64, torch.float16),
])
def test_backward_fused_launch_mixed_layouts(B, Sq, Sk, H, Hk, D, dtype):
    from flash_attn_volta import flash_attn_backward_gqa, flash_attn_forward_gqa
    print(f"[case] bwd fused mixed layouts B={B} Sq={Sq} Sk={Sk} H={H} Hk={Hk} D={D} {dtype}",
          flush=True)
    q, k, v, do = orc.make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=23, dtype=dtype)
    sc = default_scale(D, None)
    o_ref, _ = orc.attention_fwd_gqa(q, k, v, True, sc)
    dq_ref, dk_ref, dv_ref, _ = orc.attention_bwd_gqa(do, q, k, v, True, sc, o=o_ref)
    qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
    o, lse = flash_attn_forward_gqa(qd, kd, vd, causal=True, return_softmax_lse=True)
    dq, dk, dv = flash_attn_backward_gqa(dod, qd, kd, vd, o, lse, causal=True)
    tol = TOL if dtype == torch.float16 else 4e-2
    errs = dict(dq=max_abs(dq, dq_ref), dk=max_abs(dk, dk_ref), dv=max_abs(dv, dv_ref))
    report(f"bwd fused mixed {B},{Sq},{Sk},{H},{Hk},{D}", **errs)
    for key, e in errs.items():
        assert e < tol, f"{key} max-abs {e:.3e} >= {tol}"
