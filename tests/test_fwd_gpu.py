"""Forward parity on the GPU: flash_attn_forward (HIP kernel via the C ABI)
against the float64 CPU oracle on identical seeded fp16 inputs.

Mirrors the reference's forward tests (tests/test_correctness.py: max-abs
1e-2 at (2,1024,8,64), (1,2048,16,128), (4,512,4,32), both masks) and its
stability bench (bench/stability.py: S up to 8192, inputs * 0.5), and adds
every BASELINE config at full size, ragged sequence lengths, strided
(HuggingFace-transposed) inputs, D = 16, signed/zero scales and bitwise
determinism.  Tolerance: max-abs 1e-2 on O and LSE (fp16 outputs).
"""
from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from helpers import CONFIGS, TOL, default_scale, max_abs, report
from oracle import attention as orc

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=4)
def _oracle_fwd(B, S, H, D, causal, sm_scale, in_scale, seed):
    q, k, v, do = orc.make_inputs(B, S, H, D, seed=seed, scale=in_scale)
    o, lse = orc.attention_fwd(q, k, v, causal, default_scale(D, sm_scale))
    return (q, k, v, do), o, lse


def _run(q, k, v, causal, sm_scale):
    from flash_attn_volta import flash_attn_forward
    dq, dk, dv = (t.cuda() for t in (q, k, v))
    out, lse = flash_attn_forward(dq, dk, dv, causal=causal, sm_scale=sm_scale,
                                  return_softmax_lse=True)
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("cfg", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_forward_configs(cfg):
    name, B, S, H, D, causal, sm_scale, in_scale = cfg
    print(f"[case] fwd {name} B={B} S={S} H={H} D={D} causal={causal}", flush=True)
    (q, k, v, _), o_ref, lse_ref = _oracle_fwd(B, S, H, D, causal, sm_scale, in_scale, 0)
    out, lse = _run(q, k, v, causal, sm_scale)
    assert out.shape == (B, S, H, D) and out.dtype == torch.float16 and out.is_contiguous()
    assert lse.shape == (B, H, S) and lse.dtype == torch.float32
    e_o, e_l = max_abs(out, o_ref), max_abs(lse, lse_ref)
    report(f"fwd {name}", out=e_o, lse=e_l)
    assert e_o < TOL and e_l < TOL


# The reference's own forward test shapes (tests/test_correctness.py:25-29).
@pytest.mark.parametrize("shape", [(2, 1024, 8, 64), (1, 2048, 16, 128), (4, 512, 4, 32)])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_reference_shapes(shape, causal):
    B, S, H, D = shape
    print(f"[case] fwd ref-shape {shape} causal={causal}", flush=True)
    (q, k, v, _), o_ref, lse_ref = _oracle_fwd(B, S, H, D, causal, None, 1.0, 3)
    out, lse = _run(q, k, v, causal, None)
    e_o, e_l = max_abs(out, o_ref), max_abs(lse, lse_ref)
    report(f"fwd {shape} c={int(causal)}", out=e_o, lse=e_l)
    assert e_o < TOL and e_l < TOL


@pytest.mark.parametrize("S", [1, 2, 31, 33, 63, 65, 127, 129, 200, 1000])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_ragged(S, D, causal):
    B, H = 2, 3
    print(f"[case] fwd ragged S={S} D={D} causal={causal}", flush=True)
    (q, k, v, _), o_ref, lse_ref = _oracle_fwd(B, S, H, D, causal, None, 1.0, 5)
    out, lse = _run(q, k, v, causal, None)
    assert max_abs(out, o_ref) < TOL
    assert max_abs(lse, lse_ref) < TOL


# Non-causal grids of at most one 64-query workgroup per CU take the
# eight-wave layout whose query groups split each 128-key tile in four
# (fa_api.hip launch_fwd); the first shape sits at that bound (256
# workgroups), the second just past it (the two-part layout), the others
# are ragged in both lengths and use both head dims, a tile count that is
# not a multiple of the unroll and fewer keys than one tile.
@pytest.mark.parametrize("shape", [(2, 1024, 8, 64), (1, 1024, 17, 64), (3, 777, 5, 64),
                                   (1, 1000, 4, 128), (2, 100, 2, 64), (1, 1, 3, 128)])
def test_forward_four_part_layout(shape):
    B, S, H, D = shape
    print(f"[case] fwd four-part {shape}", flush=True)
    (q, k, v, _), o_ref, lse_ref = _oracle_fwd(B, S, H, D, False, None, 1.0, 7)
    out, lse = _run(q, k, v, False, None)
    e_o, e_l = max_abs(out, o_ref), max_abs(lse, lse_ref)
    report(f"fwd four-part {shape}", out=e_o, lse=e_l)
    assert e_o < TOL and e_l < TOL
    out2, lse2 = _run(q, k, v, False, None)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)


@pytest.mark.parametrize("sm_scale", [-0.125, 0.0, 0.01, 0.5])
def test_forward_signed_and_zero_scale(sm_scale):
    B, S, H, D = 1, 300, 2, 64
    print(f"[case] fwd scale={sm_scale}", flush=True)
    (q, k, v, _), o_ref, lse_ref = _oracle_fwd(B, S, H, D, True, sm_scale, 1.0, 6)
    out, lse = _run(q, k, v, True, sm_scale)
    assert max_abs(out, o_ref) < TOL
    assert max_abs(lse, lse_ref) < TOL


@pytest.mark.parametrize("D", [32, 64, 128])
def test_forward_strided_inputs_match_contiguous(D):
    """(B, H, S, D) storage viewed as (B, S, H, D) -- the HuggingFace layout --
    is read in place and gives bit-identical results."""
    from flash_attn_volta import flash_attn_forward
    B, S, H = 2, 257, 4
    print(f"[case] fwd strided D={D}", flush=True)
    q, k, v, _ = orc.make_inputs(B, S, H, D, seed=7)
    qc, kc, vc = (t.cuda() for t in (q, k, v))
    qs, ks, vs = (t.permute(0, 2, 1, 3).contiguous().cuda().transpose(1, 2) for t in (q, k, v))
    assert not qs.is_contiguous()
    for causal in (False, True):
        a, la = flash_attn_forward(qc, kc, vc, causal=causal, return_softmax_lse=True)
        b, lb = flash_attn_forward(qs, ks, vs, causal=causal, return_softmax_lse=True)
        assert torch.equal(a, b) and torch.equal(la, lb)


def test_forward_without_lse_and_determinism():
    from flash_attn_volta import flash_attn_forward, flash_attn_volta
    q, k, v, _ = orc.make_inputs(1, 1024, 4, 64, seed=8)
    q, k, v = q.cuda(), k.cuda(), v.cuda()
    out = flash_attn_forward(q, k, v, causal=True)
    assert isinstance(out, torch.Tensor)
    out2, _ = flash_attn_forward(q, k, v, causal=True, return_softmax_lse=True)
    out3 = flash_attn_volta(q, k, v, True)
    assert torch.equal(out, out2) and torch.equal(out, out3)


@pytest.mark.parametrize("shape,causal", [((1, 4096, 16, 64), False), ((1, 4096, 16, 64), True),
                                          ((1, 4096, 8, 128), False), ((1, 8192, 4, 64), False),
                                          ((1, 8192, 4, 64), True)])
def test_forward_stability_long_sequences(shape, causal):
    """Reference bench/stability.py:16-31: no NaN/Inf, inputs * 0.5."""
    from flash_attn_volta import flash_attn_forward
    B, S, H, D = shape
    print(f"[case] fwd stability {shape} causal={causal}", flush=True)
    q, k, v = orc.make_inputs(B, S, H, D, seed=9, scale=0.5, with_grad=False)
    out = flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    assert torch.isfinite(out).all()
    assert out.abs().max().item() <= v.abs().max().item() + 1e-3


def test_forward_argument_errors():
    from flash_attn_volta import flash_attn_forward
    from flash_attn_volta.forward import FlashAttnArgumentError
    q = torch.zeros(1, 8, 1, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(AssertionError):
        flash_attn_forward(q.float(), q, q)
    with pytest.raises(FlashAttnArgumentError):
        flash_attn_forward(q, q[:, :4], q)
    with pytest.raises(ValueError):
        z = torch.zeros(1, 8, 1, 48, dtype=torch.float16, device="cuda")
        flash_attn_forward(z, z, z)


# The launcher splits each tile's keys across two waves only when the grid of
# 128-query workgroups is small (< 2 per CU, < 4 causal; 256 CUs on MI355X).
# These ragged shapes are large enough to run the unsplit variant (the
# non-causal D = 64 one as eight-wave, 256-query workgroups); the shapes
# above run the split one.
@pytest.mark.parametrize("shape,causal", [((4, 1000, 32, 64), False), ((8, 1000, 32, 64), True),
                                          ((4, 777, 32, 128), False), ((8, 520, 32, 32), True)])
def test_forward_large_grid_variant(shape, causal):
    B, S, H, D = shape
    print(f"[case] fwd large-grid {shape} causal={causal}", flush=True)
    (q, k, v, _), o_ref, lse_ref = _oracle_fwd(B, S, H, D, causal, None, 1.0, 10)
    out, lse = _run(q, k, v, causal, None)
    assert max_abs(out, o_ref) < TOL
    assert max_abs(lse, lse_ref) < TOL


@pytest.mark.parametrize("causal", [False, True])
def test_forward_scores_growing_along_the_keys(causal):
    """Scores that grow steadily along the keys (K rows scaled by a ramp,
    aligned with Q): each query's running max is outgrown by ~4 (log2
    units) per 64-key tile and ~70 over the sweep, so the forward's rare
    path (take the row max, rescale O, recompute the tile) runs every few
    tiles instead of once; O and LSE must still match the oracle."""
    B, S, H, D = 1, 1024, 2, 64
    g = torch.Generator("cpu").manual_seed(40)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    ramp = torch.linspace(0.25, 6.0, S).view(1, S, 1, 1)
    q = (8.0 * u + 0.3 * torch.randn(B, S, H, D, generator=g)).half()
    k = (8.0 * ramp * u + 0.3 * torch.randn(B, S, H, D, generator=g)).half()
    v = torch.randn(B, S, H, D, generator=g).half()
    o, lse = orc.attention_fwd(q, k, v, causal, default_scale(D, None))
    out, lse_g = _run(q, k, v, causal, None)
    errs = dict(out=max_abs(out, o), lse=max_abs(lse_g, lse))
    report(f"fwd growing-scores c={int(causal)}", **errs)
    assert errs["out"] <= TOL and errs["lse"] <= TOL
