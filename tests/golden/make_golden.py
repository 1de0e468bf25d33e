"""Write tests/golden/attention_golden.npz and attention_gqa_golden.npz --
small golden vectors for the oracle.

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
from oracle.attention import make_inputs, make_inputs_gqa  # noqa: E402

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


# Grouped-query cases (attention_gqa_golden.npz).  Causal masks are aligned
# bottom-right (query i sees key j iff j <= i + Sk - Sq), written as an
# explicit boolean mask for SDPA; every case keeps at least one visible key
# per row (SDPA returns NaN for an empty row).
# name: (B, Sq, Sk, H, Hk, D, causal, sm_scale, seed)
GQA_CASES = {
    "gqa_h4_hk2_causal_sq_lt_sk": (1, 13, 29, 4, 2, 32, True, None, 10),
    "mqa_h3_hk1_sq_gt_sk": (1, 17, 9, 3, 1, 64, False, None, 11),
    "gqa_decode_sq1": (1, 1, 40, 4, 2, 64, True, None, 12),
    "gqa_square_causal_d128": (1, 16, 16, 4, 2, 128, True, 0.1, 13),
}


def golden_gqa(B, Sq, Sk, H, Hk, D, causal, sm_scale, seed):
    q, k, v, do = make_inputs_gqa(B, Sq, Sk, H, Hk, D, seed=seed)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    qf, kf, vf = (t.double().permute(0, 2, 1, 3).requires_grad_() for t in (q, k, v))
    allowed = None
    if causal:
        i = torch.arange(Sq)[:, None]
        j = torch.arange(Sk)[None, :]
        allowed = j <= i + (Sk - Sq)
    out = F.scaled_dot_product_attention(qf, kf, vf, attn_mask=allowed, scale=scale,
                                         enable_gqa=True)
    out.backward(do.double().permute(0, 2, 1, 3))
    kr = kf.detach().repeat_interleave(H // Hk, dim=1)
    s = (qf.detach() @ kr.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(~allowed, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                       # (B, H, Sq)
    perm = lambda t: t.permute(0, 2, 1, 3).contiguous().numpy()  # noqa: E731
    return {
        "q": q.numpy(), "k": k.numpy(), "v": v.numpy(), "do": do.numpy(),
        "o": perm(out.detach()), "lse": lse.numpy(),
        "dq": perm(qf.grad), "dk": perm(kf.grad), "dv": perm(vf.grad),
        "meta": np.array([B, Sq, Sk, H, Hk, D, int(causal), scale, seed], dtype=np.float64),
    }


def _write(path, cases, fn):
    arrays = {}
    for name, case in cases.items():
        for key, val in fn(*case).items():
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(path, **arrays)
    print("wrote", path, os.path.getsize(path), "bytes")


def main():
    _write(os.path.join(HERE, "attention_golden.npz"), CASES, golden)
    _write(os.path.join(HERE, "attention_gqa_golden.npz"), GQA_CASES, golden_gqa)


if __name__ == "__main__":
    main()
