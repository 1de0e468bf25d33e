"""Shared helpers for the test-suite (inputs, oracle calls, error tables)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import attention as orc

# BASELINE.json configs, as (name, B, S, H, D, causal, sm_scale, input_scale)
CONFIGS = [
    ("C1", 2, 1024, 8, 64, False, None, 1.0),
    ("C2", 4, 512, 4, 32, True, None, 1.0),
    ("C3", 1, 2048, 16, 64, True, 1.0 / 8.0, 1.0),
    ("C4a-causal", 1, 4096, 16, 64, True, None, 0.5),
    ("C4a-noncausal", 1, 4096, 16, 64, False, None, 0.5),
    ("C4b-causal", 1, 4096, 8, 128, True, None, 0.5),
    ("C4b-noncausal", 1, 4096, 8, 128, False, None, 0.5),
    ("C5-layer", 1, 4096, 16, 128, True, None, 1.0),
]

TOL = 1e-2  # max-abs, fp16 outputs vs the float64 oracle


def to_dev(*ts, device="cuda"):
    return [t.to(device) for t in ts]


def max_abs(a, b) -> float:
    a = a.detach().double().cpu().numpy() if hasattr(a, "detach") else np.asarray(a, np.float64)
    b = b.detach().double().cpu().numpy() if hasattr(b, "detach") else np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0


def default_scale(D, sm_scale):
    return 1.0 / math.sqrt(D) if sm_scale is None else sm_scale


def report(name, **errs):
    cols = " ".join(f"{k}={v:.3e}" for k, v in errs.items())
    print(f"[parity] {name:16s} {cols}", flush=True)
