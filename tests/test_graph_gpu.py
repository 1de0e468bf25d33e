"""HIP graph capture of a whole training step through flash_attn.

The C ABI neither allocates, synchronises nor records memsets (the split
backward's counters are zeroed by a kernel), and the Python wrappers
allocate through torch's caching allocator, so a forward + autograd
backward step can be captured into one graph (torch.cuda.CUDAGraph: a
hipGraph on ROCm) and replayed without Python or autograd on the host.
Every replay is checked against the eager step, with the program's own
eager work and synchronisations between the replays.
"""
from __future__ import annotations

import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,S,H,D,causal", [
    (4, 512, 4, 32, True),      # config 2: host-bound when run eagerly
    (1, 2048, 8, 128, True),    # a small causal D = 128 grid: split backward
    (2, 300, 3, 64, False),
])
def test_graph_replay_matches_eager(B, S, H, D, causal):
    from flash_attn_volta import flash_attn
    print(f"[case] graph B={B} S={S} H={H} D={D} causal={causal}", flush=True)
    q0, k0, v0, do0 = (t.cuda() for t in orc.make_inputs(B, S, H, D, seed=21))
    q, k, v = (t.clone().requires_grad_() for t in (q0, k0, v0))
    do = do0.clone()

    def step():
        q.grad = k.grad = v.grad = None
        out = flash_attn(q, k, v, causal=causal)
        out.backward(do)
        return out

    # eager reference
    ref_out = step().detach().clone()
    ref = [t.grad.clone() for t in (q, k, v)]

    # warm up on a side stream (library loads, occupancy queries, allocator)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    q.grad = k.grad = v.grad = None
    with torch.cuda.graph(g):
        out = flash_attn(q, k, v, causal=causal)
        out.backward(do)
    grads = (q.grad, k.grad, v.grad)

    for rep in range(4):
        # new inputs in place (different values on odd replays), eager work
        # between replays
        scale = 0.5 if rep % 2 else 1.0
        with torch.no_grad():
            q.copy_(q0 * scale)
        noise = torch.randn(1 << 20, device="cuda").sum()   # unrelated eager kernels
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        if scale == 1.0:
            assert torch.equal(out, ref_out), f"replay {rep}: out differs"
            for name, a, b in zip("qkv", grads, ref):
                assert torch.equal(a, b), f"replay {rep}: d{name} differs"
        else:
            # the same step on the scaled inputs, eagerly, on copies
            qe, ke, ve = (t.detach().clone().requires_grad_() for t in (q, k, v))
            oe = flash_attn(qe, ke, ve, causal=causal)
            oe.backward(do)
            assert torch.equal(out, oe.detach())
            for a, b in zip(grads, (qe.grad, ke.grad, ve.grad)):
                assert torch.equal(a, b)
