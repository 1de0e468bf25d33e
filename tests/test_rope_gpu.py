"""Fused QK-norm + rotary prologue on the GPU: rope_qk_forward /
rope_qk_backward / apply_rotary_qk (fa_rope_qk_fwd / fa_rope_qk_bwd via the
C ABI) against the float64 oracle (oracle/rope.py) on identical seeded
16-bit inputs.

Tolerance: the kernels compute in fp32 and round once, so each output may
differ from the float64 value by half a unit in the last place of its dtype
plus fp32 noise: |gpu - ref| <= 2^-10 |ref| + 1e-5 max|ref| for fp16 and
2^-7 |ref| + 1e-5 max|ref| for bf16 (twice the half-ulp bound).  The norm
weights' gradients are fp32 sums over every row: |gpu - ref| <= 1e-3
max(1, max|ref|).

Cases: Llama (no norm) and Qwen3 (q and k norms) prologues, norm on one
side only, GQA / MQA, D = 16/32/64/128, per-batch and shared cos/sin
tables, ragged row counts, the C5 layer shape, a backward grid that has to
stride over rows, fp16 and bf16; position 0 is bit-exact; strided inputs;
autograd; agreement with transformers' eager functions; determinism of the
weight gradients; argument errors.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import rope as orc

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16


def _assert_close(name, got, ref, dtype):
    g = got.detach().double().cpu().numpy()
    r = np.asarray(ref, dtype=np.float64)
    assert g.shape == r.shape, (name, g.shape, r.shape)
    rel = 2.0 ** -10 if dtype == F16 else 2.0 ** -7
    scale = float(np.max(np.abs(r))) if r.size else 0.0
    err = np.abs(g - r)
    bound = rel * np.abs(r) + 1e-5 * max(scale, 1.0)
    worst = float(np.max(err / bound)) if r.size else 0.0
    print(f"[rope] {name:8s} max_abs={float(err.max()) if r.size else 0.0:.3e} "
          f"worst/bound={worst:.3f}", flush=True)
    assert worst <= 1.0, f"{name}: error exceeds bound by {worst:.2f}x"


def _assert_dw(name, got, ref):
    g = got.detach().double().cpu().numpy()
    err = float(np.max(np.abs(g - ref)))
    print(f"[rope] {name:8s} max_abs={err:.3e} max|ref|={np.abs(ref).max():.3e}", flush=True)
    assert err <= 1e-3 * max(1.0, float(np.abs(ref).max()))


# (B, S, H, Hk, D, q_norm, k_norm, shared_table, start, dtype)
CASES = [
    (2, 37, 4, 2, 64, False, False, False, 0, F16),
    (1, 50, 8, 1, 128, True, True, False, 5, F16),
    (3, 17, 2, 2, 32, True, False, True, 1000, F16),
    (1, 9, 5, 5, 16, True, True, False, 0, F16),
    (2, 33, 6, 3, 128, False, True, False, 7, BF16),
    (1, 64, 4, 4, 64, False, False, True, 0, BF16),
    (1, 4096, 16, 16, 128, False, False, False, 0, F16),   # C5 layer, Llama
    (1, 4096, 16, 8, 128, True, True, False, 0, BF16),     # Qwen3-style at C5 size
    (1, 8192, 40, 8, 16, True, True, False, 0, F16),       # backward grid strides over rows
]


def _ids(c):
    B, S, H, Hk, D, qn, kn, sh, st, dt = c
    return f"B{B}S{S}H{H}Hk{Hk}D{D}{'-qn' if qn else ''}{'-kn' if kn else ''}" \
           f"{'-shared' if sh else ''}-{'bf16' if dt == BF16 else 'f16'}"


def _inputs(B, S, H, Hk, D, qn, kn, shared, start, dtype, seed=0):
    q, k, cos, sin, wq, wk, gq, gk = orc.make_rope_inputs(B, S, H, Hk, D, seed=seed, dtype=dtype,
                                                          norm=True, shared_table=shared,
                                                          start=start)
    return q, k, cos, sin, (wq if qn else None), (wk if kn else None), gq, gk


def _cuda(*ts):
    return [None if t is None else t.cuda() for t in ts]


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_rope_matches_oracle(case):
    from flash_attn_volta import rope_qk_backward, rope_qk_forward
    dtype = case[-1]
    eps = 1e-6
    q, k, cos, sin, wq, wk, gq, gk = _inputs(*case)
    print(f"[rope] case {_ids(case)}", flush=True)
    qd, kd, cd, sd, wqd, wkd, gqd, gkd = _cuda(q, k, cos, sin, wq, wk, gq, gk)
    qo, ko = rope_qk_forward(qd, kd, cd, sd, wqd, wkd, eps)
    dq, dk, dwq, dwk = rope_qk_backward(gqd, gkd, qd, kd, cd, sd, wqd, wkd, eps)
    torch.cuda.synchronize()
    rqo, rko = orc.rope_qk_fwd(q, k, cos, sin, wq, wk, eps)
    rdq, rdk, rdwq, rdwk = orc.rope_qk_bwd(gq, gk, q, k, cos, sin, wq, wk, eps)
    assert qo.dtype == dtype and qo.is_contiguous() and ko.is_contiguous()
    _assert_close("q_out", qo, rqo, dtype)
    _assert_close("k_out", ko, rko, dtype)
    _assert_close("dq", dq, rdq, dtype)
    _assert_close("dk", dk, rdk, dtype)
    assert (dwq is None) == (wq is None) and (dwk is None) == (wk is None)
    if wq is not None:
        assert dwq.dtype == torch.float32
        _assert_dw("dwq", dwq, rdwq)
    if wk is not None:
        _assert_dw("dwk", dwk, rdwk)


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_position_zero_is_bit_exact(dtype):
    from flash_attn_volta import rope_qk_backward, rope_qk_forward
    q, k, cos, sin, _, _, gq, gk = _inputs(2, 20, 4, 2, 128, False, False, True, 0, dtype)
    qd, kd, cd, sd, gqd, gkd = _cuda(q, k, cos, sin, gq, gk)
    qo, ko = rope_qk_forward(qd, kd, cd, sd)
    dq, dk, _, _ = rope_qk_backward(gqd, gkd, qd, kd, cd, sd)
    assert torch.equal(qo[:, 0], qd[:, 0]) and torch.equal(ko[:, 0], kd[:, 0])
    assert torch.equal(dq[:, 0], gqd[:, 0]) and torch.equal(dk[:, 0], gkd[:, 0])


def test_strided_inputs_and_table_forms():
    """q as a (B, S, H, D) view of (B, H, S, D) memory, k a head slice of a
    wider tensor, cos/sin as a 2-D (S, D) table and as fp32: bit-identical
    to the contiguous call."""
    from flash_attn_volta import rope_qk_backward, rope_qk_forward
    B, S, H, Hk, D = 2, 48, 4, 2, 64
    q, k, cos, sin, wq, wk, gq, gk = _inputs(B, S, H, Hk, D, True, True, True, 3, F16)
    qd, kd, cd, sd, wqd, wkd, gqd, gkd = _cuda(q, k, cos, sin, wq, wk, gq, gk)
    qo, ko = rope_qk_forward(qd, kd, cd, sd, wqd, wkd)
    dq, dk, dwq, dwk = rope_qk_backward(gqd, gkd, qd, kd, cd, sd, wqd, wkd)

    q_bhsd = qd.transpose(1, 2).contiguous().transpose(1, 2)       # strides (H*S*D, D, S*D, 1)
    wide = torch.zeros(B, S, Hk + 3, D, dtype=F16, device="cuda")
    wide[:, :, 1:1 + Hk] = kd
    k_sl = wide[:, :, 1:1 + Hk]
    g_bhsd = gqd.transpose(1, 2).contiguous().transpose(1, 2)
    for c2, s2 in ((cd[0], sd[0]), (cd.float(), sd.float())):
        qo2, ko2 = rope_qk_forward(q_bhsd, k_sl, c2, s2, wqd, wkd)
        dq2, dk2, dwq2, dwk2 = rope_qk_backward(g_bhsd, gkd, q_bhsd, k_sl, c2, s2, wqd, wkd)
        assert torch.equal(qo2, qo) and torch.equal(ko2, ko)
        assert torch.equal(dq2, dq) and torch.equal(dk2, dk)
        assert torch.equal(dwq2, dwq) and torch.equal(dwk2, dwk)


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_autograd_matches_oracle(dtype):
    from flash_attn_volta import apply_rotary_qk
    B, S, H, Hk, D = 2, 40, 6, 2, 128
    eps = 1e-6
    q, k, cos, sin, wq, wk, gq, gk = _inputs(B, S, H, Hk, D, True, True, False, 11, dtype)
    qd = q.cuda().requires_grad_(True)
    kd = k.cuda().requires_grad_(True)
    wqd = torch.nn.Parameter(wq.cuda())
    wkd = torch.nn.Parameter(wk.cuda())
    qo, ko = apply_rotary_qk(qd, kd, cos.cuda(), sin.cuda(), wqd, wkd, eps)
    ((qo.float() * gq.cuda().float()).sum() + (ko.float() * gk.cuda().float()).sum()).backward()
    rdq, rdk, rdwq, rdwk = orc.rope_qk_bwd(gq, gk, q, k, cos, sin, wq, wk, eps)
    _assert_close("dq", qd.grad, rdq, dtype)
    _assert_close("dk", kd.grad, rdk, dtype)
    assert wqd.grad.dtype == dtype and wkd.grad.dtype == dtype
    # the weight gradient is rounded to the weight dtype by autograd's contract
    tol = 2.0 ** -8 if dtype == F16 else 2.0 ** -6
    for got, ref in ((wqd.grad, rdwq), (wkd.grad, rdwk)):
        err = np.abs(got.double().cpu().numpy() - ref)
        assert np.all(err <= tol * np.abs(ref) + 1e-3 * max(1.0, np.abs(ref).max()))


def test_one_output_unused_in_autograd():
    from flash_attn_volta import apply_rotary_qk
    q, k, cos, sin, wq, wk, gq, gk = _inputs(1, 16, 2, 1, 64, True, False, True, 0, F16)
    qd = q.cuda().requires_grad_(True)
    kd = k.cuda().requires_grad_(True)
    qo, ko = apply_rotary_qk(qd, kd, cos.cuda(), sin.cuda(), wq.cuda(), None)
    qo.float().sum().backward()
    assert kd.grad is not None and torch.count_nonzero(kd.grad) == 0
    rdq, _, _, _ = orc.rope_qk_bwd(torch.ones_like(q), torch.zeros_like(k), q, k, cos, sin, wq,
                                   None, 1e-6)
    _assert_close("dq", qd.grad, rdq, F16)


def test_at_least_as_accurate_as_transformers_eager():
    """transformers' Qwen3RMSNorm + apply_rotary_pos_emb in fp16 on the GPU
    round after the norm, the weight product and each term of the rotation;
    the fused kernel rounds once.  Against the float64 oracle its error is
    no larger, in the worst case and on average."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb

    from flash_attn_volta import rope_qk_forward
    B, S, H, Hk, D = 1, 256, 8, 2, 128
    q, k, cos, sin, wq, wk, _, _ = _inputs(B, S, H, Hk, D, True, True, False, 0, F16)
    qd, kd, cd, sd, wqd, wkd = _cuda(q, k, cos, sin, wq, wk)
    nq, nk = Qwen3RMSNorm(D, eps=1e-6).cuda().half(), Qwen3RMSNorm(D, eps=1e-6).cuda().half()
    with torch.no_grad():
        nq.weight.copy_(wqd)
        nk.weight.copy_(wkd)
        hq, hk = apply_rotary_pos_emb(nq(qd).transpose(1, 2), nk(kd).transpose(1, 2), cd, sd)
    qo, ko = rope_qk_forward(qd, kd, cd, sd, wqd, wkd, 1e-6)
    rqo, rko = orc.rope_qk_fwd(q, k, cos, sin, wq, wk, 1e-6)
    for ours, hf, ref in ((qo, hq.transpose(1, 2), rqo), (ko, hk.transpose(1, 2), rko)):
        e_ours = np.abs(ours.double().cpu().numpy() - ref)
        e_hf = np.abs(hf.double().cpu().numpy() - ref)
        print(f"[rope] fused max={e_ours.max():.3e} mean={e_ours.mean():.3e}  "
              f"transformers max={e_hf.max():.3e} mean={e_hf.mean():.3e}", flush=True)
        assert e_ours.max() <= e_hf.max() and e_ours.mean() <= e_hf.mean()


def test_norm_weight_gradient_is_deterministic():
    from flash_attn_volta import rope_qk_backward
    q, k, cos, sin, wq, wk, gq, gk = _inputs(2, 1024, 8, 4, 128, True, True, False, 0, F16)
    args = _cuda(gq, gk, q, k, cos, sin, wq, wk)
    a = rope_qk_backward(*args)
    b = rope_qk_backward(*args)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_argument_errors():
    from flash_attn_volta import apply_rotary_qk, rope_qk_forward
    from flash_attn_volta.forward import FlashAttnArgumentError
    q, k, cos, sin, wq, wk, _, _ = _cuda(*_inputs(1, 8, 2, 1, 64, True, True, False, 0, F16))
    with pytest.raises(FlashAttnArgumentError):
        rope_qk_forward(q[..., :48].contiguous(), k[..., :48].contiguous(), cos[..., :48],
                        sin[..., :48])
    with pytest.raises(FlashAttnArgumentError):
        rope_qk_forward(q, k, cos[:, :4], sin[:, :4])
    with pytest.raises(FlashAttnArgumentError):
        rope_qk_forward(q, k.to(BF16), cos, sin)
    with pytest.raises(FlashAttnArgumentError):
        rope_qk_forward(q, k, cos, sin, wq[:32])
    with pytest.raises(FlashAttnArgumentError):
        rope_qk_forward(q.cpu(), k.cpu(), cos.cpu(), sin.cpu())
    with pytest.raises(FlashAttnArgumentError):
        apply_rotary_qk(q, k, cos.clone().requires_grad_(True), sin)
    with pytest.raises(RuntimeError):
        rope_qk_forward(q, k, cos, sin, wq, wk, eps=-1.0)
