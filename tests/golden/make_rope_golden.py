"""Write tests/golden/rope_golden.npz -- golden vectors for oracle/rope.py.

The expected values come from transformers' own ``apply_rotary_pos_emb``
(Llama's) and ``Qwen3RMSNorm`` -- the third-party functions the reference's
HF patch calls before its attention kernel (flash_attn_volta/patch_hf.py:
177, 291-303, 462) -- evaluated in float64 on the CPU, with gradients from
torch float64 autograd through them.  Tensors go in transformers' layout
(B, H, S, D) and are stored in the kernels' (B, S, H, D).  Inputs are the
seeded fp16 tensors of oracle.rope.make_rope_inputs (cos/sin as
transformers' default rotary embedding builds them), stored exactly.

    python tests/golden/make_rope_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle.rope import make_rope_inputs  # noqa: E402

# name: (B, S, H, Hk, D, q_norm, k_norm, eps, shared_table, start, seed)
CASES = {
    "llama_gqa_d64": (2, 9, 4, 2, 64, False, False, 1e-6, False, 0, 0),
    "qwen3_mqa_d128": (1, 7, 4, 1, 128, True, True, 1e-6, False, 3, 1),
    "qnorm_only_d32_shared": (2, 5, 2, 2, 32, True, False, 1e-5, True, 100, 2),
    "qwen3_d16_far": (1, 4, 3, 3, 16, True, True, 1e-6, False, 40000, 3),
}


def golden(B, S, H, Hk, D, qn, kn, eps, shared, start, seed):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    q, k, cos, sin, wq, wk, gq, gk = make_rope_inputs(B, S, H, Hk, D, seed=seed, norm=True,
                                                      shared_table=shared, start=start)
    wq = wq if qn else None
    wk = wk if kn else None
    # transformers' layout (B, H, S, D), float64, leaves for autograd
    x_q = q.double().transpose(1, 2).clone().requires_grad_(True)
    x_k = k.double().transpose(1, 2).clone().requires_grad_(True)
    params = []

    def norm(x, w):
        if w is None:
            return x
        m = Qwen3RMSNorm(D, eps=eps).double()
        with torch.no_grad():
            m.weight.copy_(w.double())
        params.append(m.weight)
        return m(x)

    yq, yk = norm(x_q, wq), norm(x_k, wk)
    oq, ok = apply_rotary_pos_emb(yq, yk, cos.double(), sin.double())
    loss = (oq * gq.double().transpose(1, 2)).sum() + (ok * gk.double().transpose(1, 2)).sum()
    loss.backward()
    out = {
        "meta": np.array([B, S, H, Hk, D, int(qn), int(kn), eps, int(shared), start, seed],
                         dtype=np.float64),
        "q": q.numpy(), "k": k.numpy(), "cos": cos.numpy(), "sin": sin.numpy(),
        "dq_out": gq.numpy(), "dk_out": gk.numpy(),
        "q_out": oq.detach().transpose(1, 2).numpy(), "k_out": ok.detach().transpose(1, 2).numpy(),
        "dq": x_q.grad.transpose(1, 2).numpy(), "dk": x_k.grad.transpose(1, 2).numpy(),
    }
    i = 0
    if wq is not None:
        out["wq"], out["dwq"] = wq.numpy(), params[i].grad.numpy()
        i += 1
    if wk is not None:
        out["wk"], out["dwk"] = wk.numpy(), params[i].grad.numpy()
    return out


def main():
    arrays = {}
    for name, args in CASES.items():
        for key, val in golden(*args).items():
            arrays[f"{name}/{key}"] = val
    path = os.path.join(HERE, "rope_golden.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, len(arrays), "arrays")


if __name__ == "__main__":
    main()
