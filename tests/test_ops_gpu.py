"""flash_attn_op (torch.library custom ops) on the GPU: the same results as
flash_attn_gqa (bit for bit: same kernels), torch.library.opcheck's schema,
fake-tensor and autograd-registration checks, and a torch.compile graph
(backend aot_eager: dynamo + AOTAutograd, no generated kernels) matching
eager outputs and gradients exactly."""
from __future__ import annotations

import pytest
import torch

from flash_attn_volta import flash_attn_gqa, flash_attn_op

pytestmark = pytest.mark.gpu


def _inputs(B, Sq, Sk, H, Hk, D, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(dtype).cuda()  # noqa: E731
    return mk(B, Sq, H, D), mk(B, Sk, Hk, D), mk(B, Sk, Hk, D), mk(B, Sq, H, D)


def _grads(fn, q, k, v, do, causal):
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    out = fn(qg, kg, vg, causal=causal)
    out.backward(do)
    torch.cuda.synchronize()
    return out.detach(), qg.grad, kg.grad, vg.grad


@pytest.mark.parametrize("case", [(2, 256, 256, 8, 8, 64, True, torch.float16),
                                  (1, 100, 300, 8, 2, 128, True, torch.bfloat16),
                                  (2, 130, 130, 4, 1, 32, False, torch.float16)])
def test_op_matches_autograd_function(case):
    B, Sq, Sk, H, Hk, D, causal, dtype = case
    print(f"[case] op {case}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hk, D, dtype, 3)
    ref = _grads(flash_attn_gqa, q, k, v, do, causal)
    got = _grads(flash_attn_op, q, k, v, do, causal)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_opcheck():
    print("[case] opcheck fwd", flush=True)
    q, k, v, _ = _inputs(1, 128, 128, 4, 2, 64, torch.float16, 5)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    torch.library.opcheck(torch.ops.flash_attn_volta.fwd.default, (q, k, v, True, 0.125),
                          test_utils=("test_schema", "test_autograd_registration",
                                      "test_faketensor"))


def test_compile_aot_eager_matches_eager():
    print("[case] torch.compile aot_eager", flush=True)

    def block(q, k, v, causal):
        return flash_attn_op(q * 1.0, k, v, causal=causal).float().square().mean()

    compiled = torch.compile(block, backend="aot_eager", fullgraph=True)
    q, k, v, _ = _inputs(2, 192, 192, 8, 4, 64, torch.float16, 7)
    res = []
    for fn in (block, compiled):
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        loss = fn(qg, kg, vg, True)
        loss.backward()
        torch.cuda.synchronize()
        res.append((loss.detach(), qg.grad, kg.grad, vg.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)
