"""Write tests/golden/attention_golden.npz -- small golden vectors for the oracle.

The expected values come from torch's own float64
``scaled_dot_product_attention`` and autograd on the CPU (a library routine
independent of oracle/), the same reference the upstream tests use
(reference tests/test_backward.py:45-56).  LSE is torch.logsumexp of the
scaled, masked float64 scores.  Inputs are the seeded fp16 tensors of
oracle.attention.make_inputs, stored as fp16.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle.attention import make_inputs  # noqa: E402

# name: (B, S, H, D, causal, sm_scale, seed)
CASES = {
    "tiny_causal_d32": (1, 16, 2, 32, True, None, 0),
    "ragged_d64": (1, 33, 1, 64, False, None, 1),
    "ragged_causal_d64": (1, 33, 1, 64, True, None, 2),
    "b2_d128_scale": (2, 12, 1, 128, True, 0.1, 3),
    "d16_causal": (1, 20, 2, 16, True, None, 4),
    "s1_d64": (1, 1, 2, 64, True, None, 5),
}


def golden(B, S, H, D, causal, sm_scale, seed):
    q, k, v, do = make_inputs(B, S, H, D, seed=seed)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    qf, kf, vf = (t.double().permute(0, 2, 1, 3).requires_grad_() for t in (q, k, v))
    out = F.scaled_dot_product_attention(qf, kf, vf, is_causal=causal, scale=scale)
    out.backward(do.double().permute(0, 2, 1, 3))
    s = (qf.detach() @ kf.detach().transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                       # (B, H, S)
    perm = lambda t: t.permute(0, 2, 1, 3).contiguous().numpy()  # noqa: E731
    return {
        "q": q.numpy(), "k": k.numpy(), "v": v.numpy(), "do": do.numpy(),
        "o": perm(out.detach()), "lse": lse.numpy(),
        "dq": perm(qf.grad), "dk": perm(kf.grad), "dv": perm(vf.grad),
        "meta": np.array([B, S, H, D, int(causal), scale, seed], dtype=np.float64),
    }


def main():
    arrays = {}
    for name, case in CASES.items():
        for key, val in golden(*case).items():
            arrays[f"{name}/{key}"] = val
    path = os.path.join(HERE, "attention_golden.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
