"""Per-shape parity record: max-abs (and mean-abs) errors of O, LSE, dQ, dK
and dV against the float64 oracle for every BASELINE config, from one run
of the current kernels on the GPU.

    python3 tests/parity_table.py            (on a GPU box, from the repo root)

The reference records the same kind of table from its tests
(tests/test_correctness.py:76-81 writes results/correctness.json, tabulated
in VERIFY.md:9-16, 136-145).  Inputs, oracle and tolerance are the ones of
tests/test_fwd_gpu.py::test_forward_configs and
tests/test_bwd_gpu.py::test_backward_configs (seeded fp16 inputs, the
float64 oracle of oracle/attention.py, max-abs 1e-2), so this prints the
numbers those tests assert on.  Prints a markdown table and a JSON block;
exits non-zero if any error reaches the tolerance.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, ROOT, os.path.join(ROOT, "flash-attn-volta_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from helpers import CONFIGS, TOL, default_scale  # noqa: E402
from oracle import attention as orc  # noqa: E402


def _errs(got, ref):
    a = got.detach().double().cpu().numpy()
    b = np.asarray(ref, np.float64)
    d = np.abs(a - b)
    return float(d.max()), float(d.mean())


def main():
    from flash_attn_volta import flash_attn_backward, flash_attn_forward
    rows = []
    for name, B, S, H, D, causal, sm_scale, in_scale in CONFIGS:
        print(f"[parity] {name} ({B},{S},{H},{D}) causal={causal} ...", file=sys.stderr, flush=True)
        q, k, v, do = orc.make_inputs(B, S, H, D, seed=0, scale=in_scale)
        sc = default_scale(D, sm_scale)
        o_ref, lse_ref = orc.attention_fwd(q, k, v, causal, sc)
        qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
        out, lse = flash_attn_forward(qd, kd, vd, causal=causal, sm_scale=sm_scale,
                                      return_softmax_lse=True)
        row = {"config": name, "shape": [B, S, H, D], "causal": causal}
        row["out"], row["out_mean"] = _errs(out, o_ref)
        row["lse"], row["lse_mean"] = _errs(lse, lse_ref)
        if name != "C1":           # C1 is the forward-only config
            dq_ref, dk_ref, dv_ref, _ = orc.attention_bwd(do, q, k, v, causal, sc, o=o_ref)
            dq, dk, dv = flash_attn_backward(dod, qd, kd, vd, out, lse, causal=causal,
                                             sm_scale=sm_scale)
            for key, got, ref in (("dq", dq, dq_ref), ("dk", dk, dk_ref), ("dv", dv, dv_ref)):
                row[key], row[key + "_mean"] = _errs(got, ref)
        torch.cuda.synchronize()
        rows.append(row)
    keys = ("out", "lse", "dq", "dk", "dv")
    print(f"| config | shape | causal | " + " | ".join(f"{k} max-abs (mean)" for k in keys) + " |")
    print("|---|---|---|" + "---:|" * len(keys))
    worst = 0.0
    for r in rows:
        cells = []
        for k in keys:
            if k in r:
                cells.append(f"{r[k]:.2e} ({r[k + '_mean']:.1e})")
                worst = max(worst, r[k])
            else:
                cells.append("-")
        print(f"| {r['config']} | {tuple(r['shape'])} | {r['causal']} | " + " | ".join(cells) + " |")
    print("\n```json")
    print(json.dumps({"tolerance_max_abs": TOL, "worst": worst, "configs": rows}, indent=1))
    print("```")
    return 0 if worst < TOL else 1


if __name__ == "__main__":
    sys.exit(main())
