"""The torch.library registrations of flash_attn_op (flash_attn_volta/ops.py)
on the CPU: the ops exist with the expected schemas, their fake-tensor
implementations give the real ops' output shapes and dtypes (grouped heads,
Sq != Sk, bf16), and a fake-mode trace keeps the attention as one node.
Nothing here runs a kernel."""
from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import flash_attn_volta  # noqa: F401  (registers the ops)
from flash_attn_volta import flash_attn_op


def test_ops_registered_with_schemas():
    fwd = torch.ops.flash_attn_volta.fwd.default
    bwd = torch.ops.flash_attn_volta.bwd.default
    assert [a.name for a in fwd._schema.arguments] == ["q", "k", "v", "causal", "sm_scale"]
    assert len(fwd._schema.returns) == 2
    assert [a.name for a in bwd._schema.arguments] == ["do", "q", "k", "v", "o", "lse",
                                                        "causal", "sm_scale"]
    assert len(bwd._schema.returns) == 3


@pytest.mark.parametrize("B,Sq,Sk,H,Hk,D,dtype", [(2, 100, 130, 8, 2, 64, torch.float16),
                                                  (1, 1, 4096, 32, 8, 128, torch.bfloat16),
                                                  (3, 77, 77, 4, 4, 32, torch.float16)])
def test_fake_shapes(B, Sq, Sk, H, Hk, D, dtype):
    with FakeTensorMode():
        q = torch.empty(B, Sq, H, D, dtype=dtype)
        k = torch.empty(B, Sk, Hk, D, dtype=dtype)
        v = torch.empty(B, Sk, Hk, D, dtype=dtype)
        out, lse = torch.ops.flash_attn_volta.fwd(q, k, v, True, 0.125)
        assert out.shape == (B, Sq, H, D) and out.dtype == dtype and out.is_contiguous()
        assert lse.shape == (B, H, Sq) and lse.dtype == torch.float32
        dq, dk, dv = torch.ops.flash_attn_volta.bwd(out, q, k, v, out, lse, True, 0.125)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
        assert dq.dtype == dk.dtype == dv.dtype == dtype


def test_fake_trace_keeps_one_node():
    def fn(q, k, v):
        return flash_attn_op(q, k, v, causal=True) * 2.0

    args = [torch.empty(1, 64, 4, 64, dtype=torch.float16) for _ in range(3)]
    g = make_fx(fn, tracing_mode="fake")(*args)
    targets = [n.target for n in g.graph.nodes if n.op == "call_function"]
    assert targets.count(torch.ops.flash_attn_volta.fwd.default) == 1
