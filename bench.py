#!/usr/bin/env python3
"""Benchmark of the hot path: FlashAttention fwd and fwd+bwd on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--prewarm-seconds T]

Workload (BASELINE.json metric): (B, S, H, D) = (1, 4096, 16, 64), causal,
fp16, synthetic N(0,1)*0.5 inputs already resident in HBM.  A step is one
``flash_attn`` forward + ``.backward(dO)`` -- the same boundary as the
reference's bench/backward.py:52-66 (autograd, delta pre-pass and all
kernels inside the timed region).  FLOPs follow the reference convention,
dense-counted even when causal: forward 4*B*H*S^2*D (bench/bench.py:69-71),
fwd+bwd 5x that (bench/backward.py:89-91).

The timed W + K steps follow a pre-warm (--prewarm-seconds, default 0.5 s
of untimed steps): the GPU raises its clocks over 0.1-0.3 s of sustained
load, and a training job runs in that state.  The same measurement taken
first, before the pre-warm, is reported beside `value` as `cold`.

Prints ONE JSON line on stdout.  `value` is the fwd+bwd TFLOP/s; the
forward-only figure, per-kernel HIP-event timings with their MFMA-roofline
fractions, and the CPU baseline (the reference's fp32 eager path, restated
in oracle/, timed on this host's cores) ride along in the same object.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_PARENT = os.path.join(ROOT, "flash-attn-volta_amd")
for _p in (ROOT, PKG_PARENT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd & fwd+bwd TFLOP/s + % fp16 MFMA peak at (1,4096,16,64) causal fp16"
PEAK_FP16_TFLOPS = 2516.6        # MI355X dense fp16 MFMA: 256 CU * 2.4 GHz * 4096 FLOP/clk
PEAK_HBM_GBS = 8000.0
B, S, H, D, CAUSAL = 1, 4096, 16, 64, True
# fa_bwd's form for this workload: causal D <= 64 backwards run the delta
# pre-pass and one fused launch of every dK/dV and dQ block
FUSED_BWD = CAUSAL and D <= 64
# Reference's published fwd+bwd figure for this exact shape and metric
# (V100-SXM2, results/backward_bench.json:65-70).
REF_FWD_BWD_TFLOPS = 61.83
REF_FWD_TFLOPS = 59.68


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def fwd_flops(b, s, h, d):
    return 4.0 * b * h * s * s * d


def causal_useful_fwd_flops(b, s, h, d):
    return 2.0 * b * h * d * s * (s + 1)


def make_inputs(device):
    import torch
    g = torch.Generator(device="cpu").manual_seed(0)
    shape = (B, S, H, D)
    q, k, v, do = (torch.randn(shape, generator=g).half().mul_(0.5).to(device) for _ in range(4))
    return q, k, v, do


def time_loop(fn, steps, warmup):
    """Wall-clock and HIP-event time of `steps` calls after `warmup` calls."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall / steps, e0.elapsed_time(e1) / 1e3 / steps


def prewarm(fn, seconds):
    """Run fn back to back for about `seconds` of wall time (synchronising
    every 20 calls).  The GPU raises its clocks over 0.1-0.3 s of sustained
    load: the same autograd step measured 236 us right after the process
    started or after 1 s idle, 202-205 us once the card had been busy
    (same box, same run).  A training job runs in the second state."""
    import torch
    t_end = time.perf_counter() + seconds
    n = 0
    while time.perf_counter() < t_end:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        n += 20
    return n


def kernel_times(q, k, v, do, steps, warmup, prewarm_s=0.0):
    """Average duration per launch of each kernel, by HIP events around
    back-to-back launches through the C ABI on torch's current stream
    (which is the stream the kernels are launched on), each loop after
    `prewarm_s` seconds of the same launches (see prewarm)."""
    import torch
    from flash_attn_volta import _capi, flash_attn_forward
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    out, lse = flash_attn_forward(q, k, v, causal=CAUSAL, return_softmax_lse=True)
    delta = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    rowmax = torch.empty(lib.fa_bwd_rowmax_bytes(B, S, H) // 4, dtype=torch.float32, device=q.device)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    st = {name: kernel_strides(t) for name, t in
          (("q", q), ("k", k), ("v", v), ("do", do), ("o", out), ("dq", dq), ("dk", dk), ("dv", dv))}
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream().cuda_stream

    def fwd():
        _capi.check(lib.fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), None,
                               B, S, H, D, st["q"], st["k"], st["v"], st["o"], scale, int(CAUSAL),
                               stream), "fa_fwd")

    def pre():
        _capi.check(lib.fa_bwd_preprocess(out.data_ptr(), do.data_ptr(), delta.data_ptr(),
                                          rowmax.data_ptr(), B, S, H, D, st["o"], st["do"], stream),
                    "fa_bwd_preprocess")

    def dkdv():
        _capi.check(lib.fa_bwd_dkdv(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    lse.data_ptr(), delta.data_ptr(), rowmax.data_ptr(),
                                    dk.data_ptr(), dv.data_ptr(),
                                    B, S, H, D, st["do"], st["q"], st["k"], st["v"], st["dk"], st["dv"],
                                    scale, int(CAUSAL), stream), "fa_bwd_dkdv")

    def dqk():
        _capi.check(lib.fa_bwd_dq(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  lse.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                  B, S, H, D, st["do"], st["q"], st["k"], st["v"], st["dq"],
                                  scale, int(CAUSAL), stream), "fa_bwd_dq")

    def blocks():
        _capi.check(lib.fa_bwd_blocks(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                      lse.data_ptr(), delta.data_ptr(), rowmax.data_ptr(),
                                      dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, S, H, D,
                                      st["do"],
                                      st["q"], st["k"], st["v"], st["dq"], st["dk"], st["dv"],
                                      scale, int(CAUSAL), stream), "fa_bwd_blocks")

    pre()
    base = 2.0 * B * H * S * S * D          # one dense S x S x D GEMM
    io = B * S * H * D * 2                  # bytes of one fp16 (B,S,H,D) tensor
    rows = B * H * S * 4                    # bytes of one fp32 (B,H,S) vector
    rmax = rows // 16                       # the row-group maxima: 2 fp32 per 32 rows
    cb = "true" if CAUSAL else "false"
    table = [
        # name, fn, kernel symbol prefix (the last template argument, the
        # in-workgroup split, is chosen by the launcher from the grid size),
        # algorithmic dense FLOPs per launch, algorithmic HBM bytes
        ("fwd", fwd, f"fa_fwd_kernel<_Float16, {D}, {cb}, ", 2 * base, 4 * io),
        ("bwd_preprocess", pre, f"fa_bwd_preprocess_kernel<_Float16, {D}>", 2.0 * B * H * S * D, 2 * io + rows + rmax),
        ("bwd_dkdv", dkdv, f"fa_bwd_dkdv_kernel<_Float16, {D}, {cb}, ", 4 * base, 6 * io + 2 * rows + rmax),
        ("bwd_dq", dqk, f"fa_bwd_dq_kernel<_Float16, {D}, {cb}, ", 3 * base, 5 * io + 2 * rows),
    ]
    if FUSED_BWD:
        # the fused launch of every dK/dV and every dQ block (fa_bwd_blocks)
        table.append(("bwd_fused", blocks, f"fa_bwd_fused_kernel<_Float16, {D}, {cb}, ",
                      7 * base, 7 * io + 2 * rows + rmax))
    res = {}
    for name, fn, sym, flops, nbytes in table:
        prewarm(fn, 0.5 * prewarm_s)
        _, ev = time_loop(fn, steps, warmup)
        res[name] = {"kernel": sym, "avg_us": ev * 1e6, "flops": flops, "bytes": nbytes,
                     "tflops": flops / ev / 1e12, "gbs": nbytes / ev / 1e9}

    # The same kernels in the training step's order with an event between
    # consecutive launches, so each kernel is timed in the step's context
    # (clock and cache state) rather than in a loop of its own: the
    # forward, then fa_bwd's launches -- the delta pre-pass and the fused
    # launch (causal D <= 64: exactly the step's launches), or the dQ and
    # dK/dV kernels (the step's dQ launch also computes delta; here delta
    # comes from the pre-pass above).
    def fwd_lse():
        _capi.check(lib.fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                               lse.data_ptr(), B, S, H, D, st["q"], st["k"], st["v"], st["o"],
                               scale, int(CAUSAL), stream), "fa_fwd")
    if FUSED_BWD:
        seq = (("fwd", fwd_lse), ("bwd_preprocess", pre), ("bwd_fused", blocks))
    else:
        seq = (("fwd", fwd_lse), ("bwd_dq", dqk), ("bwd_dkdv", dkdv))

    def seq_step():
        for _, fn in seq:
            fn()
    prewarm(seq_step, prewarm_s)
    for _ in range(warmup):
        for _, fn in seq:
            fn()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(seq) + 1)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        for j, (_, fn) in enumerate(seq):
            fn()
            ev[i][j + 1].record()
    torch.cuda.synchronize()
    # The events between launches add their own gap to each interval (a
    # few us each, about the same for every launch).  The same sequence
    # timed with events around whole steps only gives the step's true
    # length; the difference, spread evenly over the step's launches, is
    # taken off each kernel's evented interval (avg_us_in_step).  Both
    # figures are reported; the clean loop runs last, so a kernel trace of
    # this run ends with exactly these launches.
    per = {name: [ev[i][j].elapsed_time(ev[i][j + 1]) * 1e3 for i in range(steps)]
           for j, (name, _) in enumerate(seq)}
    prewarm(seq_step, 0.5 * prewarm_s)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        for _, fn in seq:
            fn()
    e1.record()
    torch.cuda.synchronize()
    step_clean = e0.elapsed_time(e1) * 1e3 / steps
    step_evented = sum(statistics.mean(v) for v in per.values())
    gap = max(0.0, (step_evented - step_clean) / len(per))
    for name, us in per.items():
        res[name]["avg_us_in_step_evented"] = statistics.mean(us)
        res[name]["median_us_in_step"] = statistics.median(us) - gap
        res[name]["avg_us_in_step"] = statistics.mean(us) - gap
        res[name]["step_us_clean"] = step_clean
        res[name]["event_gap_us"] = gap
    return res


def profiled_traffic(kernel_sym):
    """HBM bytes per launch of the kernel whose symbol starts with
    `kernel_sym`, from the committed rocprofv3 PMC summary
    (profiles/*_hbm_traffic.md: FETCH_SIZE and WRITE_SIZE runs, each scaled
    by the same counter's reading for a copy of known size).
    Returns (bytes, source, full symbol) or (None, None, kernel_sym) when no
    summary covers it."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_hbm_traffic.md"))):
        text = open(path).read()
        m = re.search(r"```json\s*(\{.*?\})\s*```", text, re.S)
        if not m:
            continue
        table = json.loads(m.group(1)).get("traffic_bytes_per_launch", {})
        for sym, nbytes in table.items():
            if sym == kernel_sym or (kernel_sym.endswith(" ") and sym.startswith(kernel_sym)):
                return float(nbytes), os.path.relpath(path, ROOT), sym
    return None, None, kernel_sym


def useful_fraction(s, causal):
    """Share of the dense-counted FLOPs that a causal kernel actually has to
    do: the score matrix's lower triangle with its diagonal, S(S+1)/2 of S^2
    entries, for every GEMM of the forward and the backward alike."""
    return (s + 1) / (2.0 * s) if causal else 1.0


# GEMMs of 2*B*H*S^2*D each that attention needs at the least: the forward's
# two (S = QK^T, O = PV) and a backward's five (S and dP recomputed once,
# dV, dK, dQ; the reference's PLAN_BACKWARD.md:8-15).  This build's backward
# issues seven: the dQ kernel and the dK/dV kernel each recompute S and dP,
# the price of writing every gradient once, without atomics.  Per backward
# kernel the shared S and dP are charged to dK/dV (S, dP, dV, dK), the dQ
# kernel keeps only its own dQ GEMM; the fused launch of both is charged the
# whole backward's five.
MINIMAL_GEMMS = {"fwd": 2, "bwd": 5, "step": 7, "bwd_dkdv": 4, "bwd_dq": 1, "bwd_fused": 5}


def minimal_flops(b, s, h, d, causal, part):
    """FLOPs of the minimal algorithm for `part` (MINIMAL_GEMMS), causal half
    (with the diagonal) when causal: the basis of every `*minimal*` figure."""
    return MINIMAL_GEMMS[part] * 2.0 * b * h * s * s * d * useful_fraction(s, causal)


def profiled_counters(kernel_sym, prefer="c4a_causal"):
    """Counter-derived figures for the kernel whose symbol starts with
    `kernel_sym`, from the committed rocprofv3 PMC summaries
    (profiles/*_counters.md, JSON block written by `bench.py --pmc-summary`),
    the benchmark workload's file (`prefer` in its name) first: the same
    kernel instantiation runs at several configs.
    Returns (dict, source) or (None, None)."""
    import glob
    import re
    paths = sorted(glob.glob(os.path.join(ROOT, "profiles", "*_counters.md")))
    for path in sorted(paths, key=lambda p: prefer not in os.path.basename(p)):
        text = open(path).read()
        m = re.search(r"```json\s*(\{.*?\})\s*```", text, re.S)
        if not m:
            continue
        table = json.loads(m.group(1)).get("kernels", {})
        for sym, row in table.items():
            if sym == kernel_sym or (kernel_sym.endswith(" ") and sym.startswith(kernel_sym)):
                return row, os.path.relpath(path, ROOT)
    return None, None


def cpu_baseline(max_seconds=30.0):
    """The reference's CPU path (ref.py eager fp32 attention, restated in
    oracle/attention.py) timed on this host: fwd+bwd through autograd on the
    full benchmark workload, 1 warmup + up to 3 timed iterations (median)."""
    import torch
    from oracle.attention import attention_ref_fp32
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(threads)
    g = torch.Generator(device="cpu").manual_seed(0)
    q, k, v, do = (torch.randn((B, S, H, D), generator=g).half().mul_(0.5) for _ in range(4))
    qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))

    def step():
        qs.grad = ks.grad = vs.grad = None
        out = attention_ref_fp32(qs, ks, vs, causal=CAUSAL)
        out.backward(do)

    t0 = time.perf_counter()
    step()
    first = time.perf_counter() - t0
    n = max(1, min(3, int(max_seconds // max(first, 1e-3))))
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": 5.0 * fwd_flops(B, S, H, D) / t / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"full workload (1,4096,16,64) causal fwd+bwd through autograd of the fp32 "
                   f"eager path; 1 warmup + {n} timed iteration(s), median {t:.2f} s"),
        "seconds_per_step": t,
        "host": {"cpu_model": model, "os_cpu_count": os.cpu_count(),
                 "affinity": len(os.sched_getaffinity(0)), "platform": platform.platform()},
    }


# BASELINE.json configs for --configs: (name, B, S, H, D, causal, sm_scale,
# input scale, fwd+bwd timed?).  C1 is the forward-only config; "C5-layer" is
# one layer of the config-5 Llama attention.
CONFIG_TABLE = [
    ("C1", 2, 1024, 8, 64, False, None, 1.0, False),
    ("C2", 4, 512, 4, 32, True, None, 1.0, True),
    ("C3", 1, 2048, 16, 64, True, 0.125, 1.0, True),
    ("C4a-causal", 1, 4096, 16, 64, True, None, 0.5, True),
    ("C4a-noncausal", 1, 4096, 16, 64, False, None, 0.5, True),
    ("C4b-causal", 1, 4096, 8, 128, True, None, 0.5, True),
    ("C4b-noncausal", 1, 4096, 8, 128, False, None, 0.5, True),
    ("C5-layer", 1, 4096, 16, 128, True, None, 1.0, True),
]


def cpu_time(fn, max_seconds):
    """1 warmup, then the median of up to 3 timed calls within ~max_seconds."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    n = max(1, min(3, int(max_seconds // max(first, 1e-3))))
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), n


def run_llama(steps, warmup):
    """one training step (causal LM loss, fwd + bwd, no
    optimizer) of a 16-layer Llama (hidden 2048, 16 heads x 128, SwiGLU
    5632, vocab 32000, random N(0, 0.02) init, fp16) at B=1, S=4096 on
    random token ids, with the attention routed to the HIP kernels by
    patch_hf (with and without the fused QK-norm / rotary prologue) and,
    for comparison, on PyTorch's own SDPA.  One JSON line per variant."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    from flash_attn_volta import patch_hf
    cfg = LlamaConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632,
                      num_hidden_layers=16, num_attention_heads=16, num_key_value_heads=16,
                      rms_norm_eps=1e-6, rope_theta=10000.0, initializer_range=0.02,
                      max_position_embeddings=4096, tie_word_embeddings=False)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = LlamaForCausalLM(cfg).half().train()
    gen = torch.Generator(device="cpu").manual_seed(5)
    ids = torch.randint(0, 32000, (1, 4096), generator=gen).cuda()
    n_params = sum(p.numel() for p in model.parameters())
    # dense training FLOPs: 6 * params * tokens for the matmuls, plus the
    # attention's 4*B*H*S^2*D per layer forward, x3 with the backward
    # (dense-counted as everywhere here)
    flops = 6.0 * n_params * 4096 + 3.0 * 16 * fwd_flops(1, 4096, 16, 128)

    def step():
        model.zero_grad(set_to_none=True)
        model(input_ids=ids, labels=ids).loss.backward()

    variants = [("patch_hf (fused rope)", lambda: patch_hf.patch_llama(model)),
                ("patch_hf", lambda: patch_hf.patch_llama(model, fuse_rope=False)),
                ("torch sdpa", lambda: 0)]
    for name, apply in variants:
        n = apply()
        _, t = time_loop(step, steps, warmup)
        row = {"config": "C5 Llama training step", "attention": name, "patched_layers": n,
               "ms_per_step": round(t * 1e3, 2), "tokens_per_s": round(4096 / t, 1),
               "model_tflops": round(flops / t / 1e12, 1), "params": n_params}
        print(json.dumps(row), flush=True)
        if n:
            patch_hf.unpatch_llama(model)


def peak_extra_bytes(step, grads):
    """Peak allocator bytes above what is allocated before one fwd+bwd step
    (inputs and dO), after a warm-up step -- the reference's measurement
    (bench/backward.py:69-85): outputs, LSE, gradients and workspace.  The
    wrappers cache the workspace per stream; it is released before the
    measured step, so the step allocates (and counts) it again."""
    import torch
    from flash_attn_volta import release_workspaces
    step()
    for t in grads:
        t.grad = None
    torch.cuda.synchronize()
    release_workspaces()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - base


def host_costs(q, k, v, do, causal, n=400):
    """Host time per call (issue time: n calls back to back, no
    synchronisation inside the timed loop) of the raw C-ABI calls with
    prepared arguments, the Python wrappers, the autograd fwd+bwd step and
    PyTorch SDPA's autograd step on the same inputs.  For a small config
    (C2) the GPU keeps up with the host, so these are host costs; the
    wrappers' overhead is wrapper minus raw call."""
    import torch
    from flash_attn_volta import _capi, flash_attn, flash_attn_backward, flash_attn_forward
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    b, s, h, d = q.shape
    sc = 1.0 / math.sqrt(d)
    out, lse = flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    stv = kernel_strides(q)
    stream = torch.cuda.current_stream().cuda_stream
    ws_bytes = lib.fa_bwd_gqa_workspace_bytes(b, s, s, h, h, d, int(causal))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    qt, kt, vt = (t.detach().transpose(1, 2).clone().requires_grad_() for t in (q, k, v))
    dot = do.transpose(1, 2).contiguous()

    def c_fwd():
        lib.fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                   b, s, h, d, stv, stv, stv, stv, sc, int(causal), stream)

    def c_bwd():
        lib.fa_bwd(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                   lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                   ws_bytes, b, s, h, d, stv, stv, stv, stv, stv, stv, stv, stv, sc, int(causal),
                   stream)

    def step():
        qg.grad = kg.grad = vg.grad = None
        flash_attn(qg, kg, vg, causal=causal).backward(do)

    def sdpa_step():
        qt.grad = kt.grad = vt.grad = None
        torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=causal).backward(dot)

    items = (("c_fwd_us", c_fwd), ("wrapper_fwd_us", lambda: flash_attn_forward(q, k, v, causal=causal)),
             ("c_bwd_us", c_bwd),
             ("wrapper_bwd_us", lambda: flash_attn_backward(do, q, k, v, out, lse, causal=causal)),
             ("autograd_step_us", step), ("sdpa_autograd_step_us", sdpa_step))
    res = {}
    for name, fn in items:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        res[name] = round((time.perf_counter() - t0) / n * 1e6, 2)
        torch.cuda.synchronize()
    res["wrapper_fwd_overhead_us"] = round(res["wrapper_fwd_us"] - res["c_fwd_us"], 2)
    res["wrapper_bwd_overhead_us"] = round(res["wrapper_bwd_us"] - res["c_bwd_us"], 2)
    return res


def steps_for(fn, steps, min_seconds=0.05):
    """`steps`, raised so the timed loop lasts about min_seconds: a short
    step (a small config's host-bound eager step) timed over 20 launches
    is mostly noise."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    per = (time.perf_counter() - t0) / 3
    return max(steps, min(2000, int(min_seconds / max(per, 1e-7))))


def run_configs(steps, warmup, with_cpu, prewarm_s=0.0):
    """Every BASELINE config: GPU forward and fwd+bwd (autograd) on the HIP
    kernels, the same fwd+bwd step replayed from a HIP graph (no host work
    per step: what small, host-bound configs reach on the GPU), and the CPU
    baseline (fp32 eager path, all host threads) for the same inputs.  One
    JSON line per config, then a markdown table."""
    import torch
    from flash_attn_volta import flash_attn, flash_attn_forward
    from oracle.attention import attention_ref_fp32
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(threads)
    rows = []
    for name, b, s, h, d, causal, sc, in_scale, with_bwd in CONFIG_TABLE:
        g = torch.Generator(device="cpu").manual_seed(0)
        qc, kc, vc = (torch.randn((b, s, h, d), generator=g).half() * in_scale for _ in range(3))
        doc = torch.randn((b, s, h, d), generator=torch.Generator(device="cpu").manual_seed(1)).half()
        q, k, v, do = (t.cuda() for t in (qc, kc, vc, doc))
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        flops = fwd_flops(b, s, h, d)

        def gpu_f():
            flash_attn_forward(q, k, v, causal=causal, sm_scale=sc)
        prewarm(gpu_f, prewarm_s)
        _, t_f = time_loop(gpu_f, steps_for(gpu_f, steps), warmup)

        def gpu_fb():
            qg.grad = kg.grad = vg.grad = None
            flash_attn(qg, kg, vg, causal=causal, sm_scale=sc).backward(do)
        t_fb = None
        if with_bwd:
            prewarm(gpu_fb, prewarm_s)
            t_fb = time_loop(gpu_fb, steps_for(gpu_fb, steps), warmup)[1]
        # the same step captured once into a HIP graph and replayed: no
        # Python / autograd work on the host per step
        t_fbg = None
        if with_bwd:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                gpu_fb()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            qg.grad = kg.grad = vg.grad = None
            with torch.cuda.graph(graph):
                flash_attn(qg, kg, vg, causal=causal, sm_scale=sc).backward(do)
            prewarm(graph.replay, prewarm_s)
            t_fbg = time_loop(graph.replay, steps_for(graph.replay, steps), warmup)[1]
            del graph
        mem = {}
        if with_bwd:
            from flash_attn_volta import backward as fa_backward
            for split in (True, False):
                fa_backward.split_workspace = split
                mem[split] = peak_extra_bytes(gpu_fb, (qg, kg, vg))
            fa_backward.split_workspace = True
        host = host_costs(q, k, v, do, causal) if name == "C2" else None
        row = {"config": name, "shape": [b, s, h, d], "causal": causal,
               "gpu_fwd_us": round(t_f * 1e6, 2), "gpu_fwd_tflops": round(flops / t_f / 1e12, 2),
               "gpu_fwd_pct_peak": round(100 * flops / t_f / 1e12 / PEAK_FP16_TFLOPS, 2)}
        useful = useful_fraction(s, causal)
        row["gpu_fwd_issued_pct"] = round(100 * useful * flops / t_f / 1e12 / PEAK_FP16_TFLOPS, 2)
        if with_bwd:
            row.update({"gpu_fwd_bwd_us": round(t_fb * 1e6, 2),
                        "gpu_fwd_bwd_tflops": round(5 * flops / t_fb / 1e12, 2),
                        "gpu_fwd_bwd_pct_peak": round(100 * 5 * flops / t_fb / 1e12 / PEAK_FP16_TFLOPS, 2),
                        # 9 GEMMs issued (2 fwd + 7 bwd), 7 minimal, causal half
                        "gpu_fwd_bwd_issued_pct": round(
                            100 * 4.5 * useful * flops / t_fb / 1e12 / PEAK_FP16_TFLOPS, 2),
                        "gpu_fwd_bwd_minimal_pct": round(
                            100 * minimal_flops(b, s, h, d, causal, "step") / t_fb / 1e12
                            / PEAK_FP16_TFLOPS, 2),
                        "gpu_fwd_bwd_graph_us": round(t_fbg * 1e6, 2),
                        "gpu_fwd_bwd_graph_tflops": round(5 * flops / t_fbg / 1e12, 2),
                        "peak_extra_mb": round(mem[True] / 1e6, 2),
                        "peak_extra_mb_no_split": round(mem[False] / 1e6, 2)})
        if host is not None:
            row["host"] = host
        if with_cpu:
            with torch.no_grad():
                t_cf, n_f = cpu_time(lambda: attention_ref_fp32(qc, kc, vc, causal=causal, sm_scale=sc), 10.0)
            row.update({"cpu_fwd_tflops": round(flops / t_cf / 1e12, 4), "cpu_threads": torch.get_num_threads()})
            if with_bwd:
                qs, ks, vs = (t.clone().requires_grad_() for t in (qc, kc, vc))

                def cpu_fb():
                    qs.grad = ks.grad = vs.grad = None
                    attention_ref_fp32(qs, ks, vs, causal=causal, sm_scale=sc).backward(doc)
                t_cfb, _ = cpu_time(cpu_fb, 10.0)
                row["cpu_fwd_bwd_tflops"] = round(5 * flops / t_cfb / 1e12, 4)
        rows.append(row)
        print(json.dumps(row), flush=True)
    hdr = ("| config | shape | GPU fwd us | GPU fwd TFLOP/s (% peak; % issued) | GPU fwd+bwd us | "
           "GPU fwd+bwd TFLOP/s (% peak; % issued; % minimal) | fwd+bwd graph replay us (TFLOP/s) | "
           "peak extra MB (no split) | CPU fwd TFLOP/s | CPU fwd+bwd TFLOP/s |")
    print(hdr)
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        fb = (f"{r['gpu_fwd_bwd_us']} | {r['gpu_fwd_bwd_tflops']} ({r['gpu_fwd_bwd_pct_peak']} %; "
              f"{r['gpu_fwd_bwd_issued_pct']} %; {r['gpu_fwd_bwd_minimal_pct']} %) | "
              f"{r['gpu_fwd_bwd_graph_us']} ({r['gpu_fwd_bwd_graph_tflops']}) | "
              f"{r['peak_extra_mb']} ({r['peak_extra_mb_no_split']})"
              if "gpu_fwd_bwd_us" in r else "n/a | n/a | n/a | n/a")
        print(f"| {r['config']} | {tuple(r['shape'])}{' causal' if r['causal'] else ''} | "
              f"{r['gpu_fwd_us']} | {r['gpu_fwd_tflops']} ({r['gpu_fwd_pct_peak']} %; "
              f"{r['gpu_fwd_issued_pct']} %) | {fb} | "
              f"{r.get('cpu_fwd_tflops', '-')} | {r.get('cpu_fwd_bwd_tflops', '-')} |")


# Grids several rounds of workgroups deep, for --large: (B, S, H, D, causal)
LARGE_TABLE = [
    (4, 4096, 16, 64, False),
    (4, 4096, 16, 64, True),
    (4, 4096, 16, 128, False),
    (4, 4096, 16, 128, True),
    (1, 16384, 16, 128, True),
]


def run_large(steps, warmup, prewarm_s=0.0):
    """Forward and backward calls (flash_attn_forward with LSE,
    flash_attn_backward) on grids that fill the GPU several times over,
    inputs N(0, 1) * 0.5, pre-warmed, HIP events.  TFLOP/s in the metric's
    convention (forward 4*B*H*S^2*D, backward 4x that, dense when causal);
    `issued_pct` is the share of the MFMA peak spent on the work the kernels
    issue: half the scores when causal, and 7 GEMMs of 2*S^2*D per head in
    the backward (S and dP recomputed by both backward kernels), 3.5x the
    forward's 2.  One JSON line per shape, then a markdown table."""
    import torch
    from flash_attn_volta import flash_attn_backward, flash_attn_forward
    rows = []
    for b, s, h, d, causal in LARGE_TABLE:
        g = torch.Generator(device="cpu").manual_seed(0)
        q, k, v, do = (torch.randn((b, s, h, d), generator=g).half().mul_(0.5).cuda()
                       for _ in range(4))
        o, lse = flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)

        def fwd():
            flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)

        def bwd():
            flash_attn_backward(do, q, k, v, o, lse, causal=causal)
        flops = fwd_flops(b, s, h, d)
        useful = 0.5 if causal else 1.0
        row = {"shape": [b, s, h, d], "causal": causal}
        for name, fn, counted, issued in (("fwd", fwd, 1.0, 1.0), ("bwd", bwd, 4.0, 3.5)):
            prewarm(fn, prewarm_s)
            t = time_loop(fn, steps, warmup)[1]
            row[f"{name}_us"] = round(t * 1e6, 2)
            row[f"{name}_tflops"] = round(counted * flops / t / 1e12, 1)
            row[f"{name}_issued_pct"] = round(
                100 * issued * useful * flops / t / 1e12 / PEAK_FP16_TFLOPS, 1)
            row[f"{name}_minimal_pct"] = round(
                100 * minimal_flops(b, s, h, d, causal, name) / t / 1e12 / PEAK_FP16_TFLOPS, 1)
        rows.append(row)
        print(json.dumps(row), flush=True)
    print("| (B,S,H,D) | fwd us | fwd TFLOP/s (issued % of peak) | bwd us | "
          "bwd TFLOP/s (issued % of peak; minimal 5-GEMM % of peak) |")
    print("|---|---:|---:|---:|---:|")
    for r in rows:
        print(f"| {tuple(r['shape'])}{' causal' if r['causal'] else ' non-causal'} | "
              f"{r['fwd_us']} | {r['fwd_tflops']} ({r['fwd_issued_pct']} %) | "
              f"{r['bwd_us']} | {r['bwd_tflops']} ({r['bwd_issued_pct']} %; "
              f"{r['bwd_minimal_pct']} %) |")


# Fused-prologue workloads: (name, B, S, H, Hk, D, qk_norm, dtype name)
ROPE_TABLE = [
    ("C5-llama", 1, 4096, 16, 16, 128, False, "fp16"),
    ("C5-qwen3", 1, 4096, 16, 8, 128, True, "bf16"),
]


def rope_bytes(b, s, h, hk, d, norm, tables_b=1):
    """Algorithmic HBM bytes of the fused prologue's forward and backward
    launches: each q/k element read and written once (16-bit), the forward
    inputs read again by a normed backward, the cos/sin tables once, and the
    backward's fp32 dw partials written and read."""
    elems = b * s * (h + hk) * d
    tables = 2 * tables_b * s * d * 2
    fwd = 2 * elems * 2 + tables
    bwd = 2 * elems * 2 + tables
    if norm:
        rows = b * s * max(h, hk)
        nblk = min(-(-rows // (4096 // d)), 1024)
        bwd += elems * 2 + 2 * (2 * nblk * d * 4)
    return fwd, bwd


def rope_kernel_times(q, k, cos, sin, wq, wk, gq, gk, eps, steps, warmup):
    """Average HIP-event time per call of fa_rope_qk_fwd and fa_rope_qk_bwd
    (the backward including its dw reduction), launched back to back through
    the C ABI with prepared arguments, so the host issues faster than the
    GPU drains."""
    import torch
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import _DTYPES, kernel_strides
    lib = _capi.load()
    b, s, h, d = q.shape
    hk = k.shape[2]
    qo, ko, dq, dk = (torch.empty_like(t) for t in (q, k, q, k))
    dwq = torch.empty(d, dtype=torch.float32, device=q.device) if wq is not None else None
    dwk = torch.empty(d, dtype=torch.float32, device=q.device) if wk is not None else None
    ws = torch.empty(lib.fa_rope_qk_workspace_bytes(b, s, h, hk, d), dtype=torch.uint8,
                     device=q.device)
    cs = (ctypes.c_int64 * 2)(0, d)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    stream = torch.cuda.current_stream().cuda_stream
    dt = _DTYPES[q.dtype]
    fa = (ptr(q), ptr(k), ptr(qo), ptr(ko), ptr(cos), ptr(sin), ptr(wq), ptr(wk), eps,
          b, s, h, hk, d, kernel_strides(q), kernel_strides(k), kernel_strides(qo),
          kernel_strides(ko), cs, dt, stream)
    ba = (ptr(gq), ptr(gk), ptr(q), ptr(k), ptr(cos), ptr(sin), ptr(wq), ptr(wk), eps,
          ptr(dq), ptr(dk), ptr(dwq), ptr(dwk), ptr(ws), ws.numel(), b, s, h, hk, d,
          kernel_strides(gq), kernel_strides(gk), kernel_strides(q), kernel_strides(k),
          kernel_strides(dq), kernel_strides(dk), cs, dt, stream)
    out = []
    for fn, a in ((lib.fa_rope_qk_fwd, fa), (lib.fa_rope_qk_bwd, ba)):
        _capi.check(fn(*a), "rope kernel timing")
        out.append(time_loop(lambda: fn(*a), steps, warmup)[1])
    return out


def run_rope(steps, warmup):
    """The fused QK-norm + rotary prologue against transformers' eager
    prologue (Qwen3RMSNorm + apply_rotary_pos_emb, as the reference's patch
    calls them) at the config-5 layer shape: kernel times and HBM roofline
    of fa_rope_qk_fwd / fa_rope_qk_bwd, and fwd / fwd+bwd of both prologues
    through autograd, next to the attention fwd+bwd of the same layer."""
    import torch
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb
    from flash_attn_volta import apply_rotary_qk, flash_attn_gqa
    rows = []
    for name, b, s, h, hk, d, norm, dt in ROPE_TABLE:
        dtype = torch.float16 if dt == "fp16" else torch.bfloat16
        g = torch.Generator(device="cpu").manual_seed(0)
        q, gq = (torch.randn((b, s, h, d), generator=g).to(dtype).cuda() for _ in range(2))
        k, gk = (torch.randn((b, s, hk, d), generator=g).to(dtype).cuda() for _ in range(2))
        # rotary tables as transformers' default rotary embedding builds them
        inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
        freqs = torch.arange(s).float()[:, None] * inv
        emb = torch.cat((freqs, freqs), dim=-1)[None]
        cos, sin = emb.cos().to(dtype).cuda(), emb.sin().to(dtype).cuda()
        wq = wk = None
        if norm:
            wq, wk = ((1.0 + 0.25 * torch.randn(d, generator=g)).to(dtype).cuda() for _ in range(2))
        eps = 1e-6
        t_kf, t_kb = rope_kernel_times(q, k, cos, sin, wq, wk, gq, gk, eps, steps, warmup)
        by_f, by_b = rope_bytes(b, s, h, hk, d, norm)

        qg, kg = q.clone().requires_grad_(), k.clone().requires_grad_()
        wqg = torch.nn.Parameter(wq.clone()) if norm else None
        wkg = torch.nn.Parameter(wk.clone()) if norm else None
        nq = nk = None
        if norm:
            nq, nk = Qwen3RMSNorm(d, eps=eps).cuda().to(dtype), Qwen3RMSNorm(d, eps=eps).cuda().to(dtype)
            with torch.no_grad():
                nq.weight.copy_(wq)
                nk.weight.copy_(wk)

        def fused_fb():
            qg.grad = kg.grad = None
            qo, ko = apply_rotary_qk(qg, kg, cos, sin, wqg, wkg, eps)
            torch.autograd.backward((qo, ko), (gq, gk))

        def hf_prologue(qx, kx):
            if norm:
                qx, kx = nq(qx), nk(kx)
            return apply_rotary_pos_emb(qx.transpose(1, 2), kx.transpose(1, 2), cos, sin)

        def hf_fb():
            qg.grad = kg.grad = None
            qo, ko = hf_prologue(qg, kg)
            torch.autograd.backward((qo, ko), (gq.transpose(1, 2), gk.transpose(1, 2)))

        with torch.no_grad():
            _, t_ff = time_loop(lambda: apply_rotary_qk(q, k, cos, sin, wq, wk, eps), steps, warmup)
            _, t_hf = time_loop(lambda: hf_prologue(q, k), steps, warmup)
        _, t_ffb = time_loop(fused_fb, steps, warmup)
        _, t_hfb = time_loop(hf_fb, steps, warmup)
        v = torch.randn_like(k)
        qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
        do = torch.randn_like(q)

        def attn_fb():
            qa.grad = ka.grad = va.grad = None
            flash_attn_gqa(qa, ka, va, causal=True).backward(do)
        _, t_att = time_loop(attn_fb, steps, warmup)
        row = {"workload": name, "shape": [b, s, h, hk, d], "qk_norm": norm, "dtype": dt,
               "kernel_fwd_us": round(t_kf * 1e6, 2),
               "kernel_fwd_gbs": round(by_f / t_kf / 1e9, 1),
               "kernel_fwd_frac_hbm": round(by_f / t_kf / 1e9 / PEAK_HBM_GBS, 4),
               "kernel_bwd_us": round(t_kb * 1e6, 2),
               "kernel_bwd_gbs": round(by_b / t_kb / 1e9, 1),
               "kernel_bwd_frac_hbm": round(by_b / t_kb / 1e9 / PEAK_HBM_GBS, 4),
               "algorithmic_bytes": {"fwd": by_f, "bwd": by_b},
               "fused_fwd_us": round(t_ff * 1e6, 2), "transformers_fwd_us": round(t_hf * 1e6, 2),
               "fused_fwd_bwd_us": round(t_ffb * 1e6, 2),
               "transformers_fwd_bwd_us": round(t_hfb * 1e6, 2),
               "speedup_fwd_bwd": round(t_hfb / t_ffb, 2),
               "attention_fwd_bwd_us": round(t_att * 1e6, 2)}
        rows.append(row)
        print(json.dumps(row), flush=True)
    print("| workload | shape (B,S,H,Hk,D) | kernel fwd us (GB/s, % of 8 TB/s) | kernel bwd us "
          "(GB/s, %) | fused fwd+bwd us | transformers fwd+bwd us | speed-up | attention "
          "fwd+bwd us |")
    print("|---|---|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        print(f"| {r['workload']} ({r['dtype']}{', qk-norm' if r['qk_norm'] else ''}) | "
              f"{tuple(r['shape'])} | {r['kernel_fwd_us']} ({r['kernel_fwd_gbs']}, "
              f"{100 * r['kernel_fwd_frac_hbm']:.1f} %) | {r['kernel_bwd_us']} ({r['kernel_bwd_gbs']}, "
              f"{100 * r['kernel_bwd_frac_hbm']:.1f} %) | {r['fused_fwd_bwd_us']} | "
              f"{r['transformers_fwd_bwd_us']} | {r['speedup_fwd_bwd']}x | "
              f"{r['attention_fwd_bwd_us']} |")


# Decode workloads (one new token, or a few, against a KV cache), fp16,
# causal: (B, Sq, Sk, H, Hk, D)
DECODE_TABLE = [
    (1, 1, 4096, 32, 8, 128),
    (1, 1, 32768, 32, 8, 128),
    (1, 1, 131072, 64, 8, 128),
    (8, 1, 8192, 32, 8, 128),
    (4, 4, 8192, 32, 8, 128),
    (1, 1, 8192, 32, 32, 128),
    (1, 1, 4096, 16, 16, 64),
]


def run_decode(steps, warmup):
    """Decode-step attention: fa_fwd_splitkv (keys split over workgroups,
    partials merged by LSE) against the unsplit fa_fwd_gqa on the same
    inputs, by HIP events around back-to-back C-ABI launches.  Algorithmic
    bytes = K and V read once + Q read + O written (+ LSE); HBM-bound."""
    import torch
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    rows = []
    for (b, sq, sk, h, hk, d) in DECODE_TABLE:
        g = torch.Generator(device="cpu").manual_seed(0)
        q = torch.randn((b, sq, h, d), generator=g).half().cuda()
        k, v = (torch.randn((b, sk, hk, d), generator=g).half().cuda() for _ in range(2))
        o = torch.empty_like(q)
        lse = torch.empty((b, h, sq), dtype=torch.float32, device="cuda")
        st = [kernel_strides(t) for t in (q, k, v, o)]
        stream = torch.cuda.current_stream().cuda_stream
        nb = lib.fa_fwd_splitkv_workspace_bytes(b, sq, sk, h, hk, d)
        ws = torch.empty(max(nb, 256), dtype=torch.uint8, device="cuda")
        common = (b, sq, sk, h, hk, d, *st, d ** -0.5, 1, _capi.FA_DTYPE_F16, stream)
        ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr())
        unsplit = lambda: lib.fa_fwd_gqa(*ptrs, *common)  # noqa: E731
        split = lambda: lib.fa_fwd_splitkv(*ptrs, ws.data_ptr(), ws.numel(), *common)  # noqa: E731
        _capi.check(split(), "fa_fwd_splitkv")
        t_u = time_loop(unsplit, steps, warmup)[1]
        t_s = time_loop(split, steps, warmup)[1]
        by = 2 * b * sk * hk * d * 2 + 2 * b * sq * h * d * 2 + b * h * sq * 4
        row = {"shape": [b, sq, sk, h, hk, d], "workspace_bytes": nb,
               "unsplit_us": round(t_u * 1e6, 2), "splitkv_us": round(t_s * 1e6, 2),
               "algorithmic_bytes": by, "splitkv_gbs": round(by / t_s / 1e9, 1),
               "splitkv_frac_hbm": round(by / t_s / 1e9 / PEAK_HBM_GBS, 4),
               "speedup": round(t_u / t_s, 2)}
        rows.append(row)
        print(json.dumps(row), flush=True)
    print("| (B, Sq, Sk, H, Hk, D) | unsplit us | split-KV us | split-KV GB/s (% of 8 TB/s) | speed-up |")
    print("|---|---:|---:|---:|---:|")
    for r in rows:
        print(f"| {tuple(r['shape'])} | {r['unsplit_us']} | {r['splitkv_us']} | {r['splitkv_gbs']} "
              f"({100 * r['splitkv_frac_hbm']:.1f} %) | {r['speedup']}x |")


def run_profile_config(name, steps, warmup, prewarm_s=0.0):
    """The training step's kernels for one BASELINE config, as the program
    that rocprofv3 counter passes run: `warmup` + `steps` rounds of
    flash_attn_forward (with LSE) and flash_attn_backward on the same
    inputs as --configs, nothing else on the GPU in between (with
    `prewarm_s` > 0, first that long of the same rounds, so that a kernel
    trace's averages are dominated by launches at ramped clocks)."""
    import torch
    from flash_attn_volta import flash_attn_backward, flash_attn_forward
    rows = [r for r in CONFIG_TABLE if r[0] == name]
    if not rows:
        raise SystemExit(f"unknown config {name!r}; one of {[r[0] for r in CONFIG_TABLE]}")
    _, b, s, h, d, causal, sc, in_scale, _ = rows[0]
    g = torch.Generator(device="cpu").manual_seed(0)
    q, k, v = (((torch.randn((b, s, h, d), generator=g)).half() * in_scale).cuda() for _ in range(3))
    do = torch.randn((b, s, h, d), generator=torch.Generator(device="cpu").manual_seed(1)).half().cuda()
    def rnd():
        o, lse = flash_attn_forward(q, k, v, causal=causal, sm_scale=sc, return_softmax_lse=True)
        flash_attn_backward(do, q, k, v, o, lse, causal=causal, sm_scale=sc)
    if prewarm_s > 0:
        prewarm(rnd, prewarm_s)
    for _ in range(warmup + steps):
        rnd()
    torch.cuda.synchronize()
    log(f"[bench] profiled {name} ({b},{s},{h},{d}) causal={causal}: {warmup + steps} steps")


def demangle_fa(name):
    """`fa_fwd_kernel<_Float16, 64, true, 2, false>` for this library's
    kernel symbols, mangled (`_ZN2fa13fa_fwd_kernelIDF16_Li64ELb1E...`, as
    some rocprofv3 outputs give them; binutils' c++filt does not know the
    _Float16 mangling) or demangled (`void fa::fa_fwd_kernel<...>(...)`)."""
    import re
    if not name.startswith("_ZN2fa"):
        return name.replace("void ", "").replace("fa::", "").split("(")[0].strip()
    m = re.match(r"_ZN2fa(\d+)", name)
    n = int(m.group(1))
    pos = m.end()
    kname = name[pos:pos + n]
    pos += n
    args = []
    if name[pos:pos + 1] == "I":
        pos += 1
        tokens = [(r"DF16_", "_Float16"), (r"DF16b", "__bf16"), (r"Li(-?\d+)E", None),
                  (r"Lb([01])E", None)]
        while pos < len(name) and name[pos] != "E":
            for pat, text in tokens:
                t = re.match(pat, name[pos:])
                if t:
                    if text is not None:
                        args.append(text)
                    elif pat.startswith("Lb"):
                        args.append("true" if t.group(1) == "1" else "false")
                    else:
                        args.append(t.group(1))
                    pos += t.end()
                    break
            else:
                return name          # not one of ours: leave it
    return f"{kname}<{', '.join(args)}>" if args else kname


# rocprofv3 --pmc passes summarised by --pmc-summary (each within the
# per-pass limits: at most 8 SQ and 2 GRBM counters)
PMC_PASSES = {
    "A": "SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_LDS "
         "SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_VALU_TRANS_F32 GRBM_GUI_ACTIVE",
    "B": "SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY "
         "SQ_ACTIVE_INST_VALU SQ_VALU_MFMA_COEXEC_CYCLES SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE",
}
XCDS = 8            # MI355X: GRBM_GUI_ACTIVE comes back summed over the 8 XCDs
CUS = 256
SIMDS = 4 * CUS     # 256 CUs x 4 SIMDs


def pmc_summary(dirs):
    """Per-kernel averages of rocprofv3 --pmc counter_collection.csv files
    (one directory per pass) for the fa:: kernels, with the derived figures:

      mfma_busy   = SQ_VALU_MFMA_BUSY_CYCLES / (cycles * SIMDS), cycles =
                    GRBM_GUI_ACTIVE / XCDS (rocprofiler's MfmaUtil);
      *_per_mfma  = instruction counts per MFMA instruction (VALU excludes
                    the MFMAs, which SQ_INSTS_VALU counts among its own);
      lds_bank_conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE;
      waves_per_simd = SQ_WAVE_CYCLES * 4 / (cycles * SIMDS) (wave-cycles
                    come in quad-cycles): mean resident waves per SIMD;
      wait_any, wait_issue, active = SQ_WAIT_ANY, SQ_WAIT_INST_ANY,
                    SQ_ACTIVE_INST_ANY as shares of SQ_WAVE_CYCLES;
      mfma_coexec = SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES
                    (share of MFMA-busy cycles in which a VALU op issued);
      lds_latency, vmem_latency = rocprofiler's LdsLatency / VmemLatency
                    (in-flight instruction level accumulated per cycle over
                    the instruction count: mean cycles from issue to data);
      iss_valu, iss_lds, iss_sca, iss_misc, iss_vmem, wait_lds =
                    SQ_ACTIVE_INST_{VALU,LDS,SCA,MISC,VMEM} and
                    SQ_WAIT_INST_LDS as shares of SQ_WAVE_CYCLES (VALU
                    includes the MFMAs; SCA = SALU + SMEM; MISC = branches,
                    barriers and messages).

    Prints a markdown table and the JSON block that bench.py reads back
    (profiles/*_counters.md)."""
    import collections
    import csv
    import glob
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    meta = {}
    for dr in dirs:
        for path in glob.glob(os.path.join(dr, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                name = r["Kernel_Name"]
                if "fa_" not in name:
                    continue
                vals[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
                meta[name] = {"grid": int(r["Grid_Size"]), "workgroup": int(r["Workgroup_Size"]),
                              "lds_bytes": int(r["LDS_Block_Size"])}
    out = {}
    for raw in sorted(vals):
        key = demangle_fa(raw)
        av = {c: statistics.mean(v) for c, v in vals[raw].items()}
        cyc = av.get("GRBM_GUI_ACTIVE", 0.0) / XCDS
        row = dict(meta[raw])
        row["cycles"] = round(cyc)
        mf = av.get("SQ_INSTS_MFMA")
        if cyc and "SQ_VALU_MFMA_BUSY_CYCLES" in av:
            row["mfma_busy"] = round(av["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * SIMDS), 4)
        if mf:
            row["mfma_insts"] = round(mf)
            if "SQ_INSTS_VALU" in av:
                row["valu_per_mfma"] = round((av["SQ_INSTS_VALU"] - mf) / mf, 3)
            for c, k in (("SQ_INSTS_SALU", "salu_per_mfma"), ("SQ_INSTS_LDS", "lds_per_mfma"),
                         ("SQ_INSTS_VALU_TRANS_F32", "trans_per_mfma")):
                if c in av:
                    row[k] = round(av[c] / mf, 3)
        if av.get("SQ_LDS_IDX_ACTIVE"):
            row["lds_bank_conflict"] = round(av["SQ_LDS_BANK_CONFLICT"] / av["SQ_LDS_IDX_ACTIVE"], 4)
        wc = av.get("SQ_WAVE_CYCLES")
        if wc and cyc:
            row["waves_per_simd"] = round(wc * 4 / (cyc * SIMDS), 3)
            for c, k in (("SQ_WAIT_ANY", "wait_any"), ("SQ_WAIT_INST_ANY", "wait_issue"),
                         ("SQ_ACTIVE_INST_ANY", "active")):
                if c in av:
                    row[k] = round(av[c] / wc, 4)
        if wc:
            for c, k in (("SQ_ACTIVE_INST_VALU", "iss_valu"), ("SQ_ACTIVE_INST_LDS", "iss_lds"),
                         ("SQ_ACTIVE_INST_SCA", "iss_sca"), ("SQ_ACTIVE_INST_MISC", "iss_misc"),
                         ("SQ_ACTIVE_INST_VMEM", "iss_vmem"), ("SQ_WAIT_INST_LDS", "wait_lds")):
                if c in av:
                    row[k] = round(av[c] / wc, 4)
        for c, k in (("LdsLatency", "lds_latency"), ("VmemLatency", "vmem_latency")):
            if c in av:
                row[k] = round(av[c], 1)
        if av.get("SQ_VALU_MFMA_BUSY_CYCLES") and "SQ_VALU_MFMA_COEXEC_CYCLES" in av:
            row["mfma_coexec"] = round(av["SQ_VALU_MFMA_COEXEC_CYCLES"] / av["SQ_VALU_MFMA_BUSY_CYCLES"], 4)
        # the texture / LDS pass (one TA and one TD per CU; LDS load
        # bandwidth in 64-byte units, summed over the CUs)
        if cyc:
            if "TA_TA_BUSY" in av:
                row["ta_busy"] = round(av["TA_TA_BUSY"] / (cyc * CUS), 4)
            if "TD_TD_BUSY" in av:
                row["td_busy"] = round(av["TD_TD_BUSY"] / (cyc * CUS), 4)
            if "TD_TC_STALL" in av:
                row["td_tc_stall"] = round(av["TD_TC_STALL"] / (cyc * CUS), 4)
            if "SQ_INSTS_LDS_LOAD_BANDWIDTH" in av:
                row["lds_load_b_per_clk_cu"] = round(64.0 * av["SQ_INSTS_LDS_LOAD_BANDWIDTH"] / (cyc * CUS), 1)
        out[key] = row
    cols = ["cycles", "mfma_busy", "valu_per_mfma", "salu_per_mfma", "lds_per_mfma", "trans_per_mfma",
            "lds_bank_conflict", "waves_per_simd", "wait_any", "wait_issue", "active", "mfma_coexec",
            "ta_busy", "td_busy", "td_tc_stall", "lds_load_b_per_clk_cu",
            "iss_valu", "iss_lds", "iss_sca", "iss_misc", "iss_vmem", "wait_lds",
            "lds_latency", "vmem_latency",
            "lds_bytes", "grid", "workgroup"]
    cols = [c for c in cols if any(c in r for r in out.values())]
    print("| kernel | " + " | ".join(cols) + " |")
    print("|---|" + "---:|" * len(cols))
    for key, row in out.items():
        print(f"| `{key}` | " + " | ".join(str(row.get(c, "")) for c in cols) + " |")
    print("\n```json")
    print(json.dumps({"kernels": out, "xcds": XCDS, "simds": SIMDS}, indent=1))
    print("```")


def traffic_summary(dirs):
    """HBM bytes per launch from four rocprofv3 --pmc output directories:
    FETCH_SIZE and WRITE_SIZE over the benchmark's kernels, then the same two
    counters over --copy-calibration's plain device copies, whose known
    traffic (read n + write n bytes per dispatch) gives the scale of each
    counter.  Prints the per-kernel table and the JSON block that
    profiled_traffic() reads back (profiles/*_hbm_traffic.md)."""
    import collections
    import csv
    import glob

    def per_kernel(dr, counter):
        vals = collections.defaultdict(list)
        for path in glob.glob(os.path.join(dr, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if r["Counter_Name"] == counter:
                    vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
        return {k: statistics.mean(v) for k, v in vals.items()}

    fetch, write = per_kernel(dirs[0], "FETCH_SIZE"), per_kernel(dirs[1], "WRITE_SIZE")
    cfetch, cwrite = per_kernel(dirs[2], "FETCH_SIZE"), per_kernel(dirs[3], "WRITE_SIZE")
    copy = [k for k in cfetch if "copyBuffer" in k or "copy" in k.lower()]
    if not copy:
        raise SystemExit("no copy kernel in the calibration runs")
    # the calibration copy reads and writes n bytes; WRITE_SIZE counts the
    # write exactly (scale 1), FETCH_SIZE is scaled to the same n
    n_kib = cwrite[copy[0]]
    f_scale = n_kib / cfetch[copy[0]]
    w_scale = n_kib / cwrite[copy[0]]
    print(f"Calibration: the copy writes {n_kib:.1f} KiB per dispatch: FETCH_SIZE reads "
          f"{cfetch[copy[0]]:.1f} KiB, WRITE_SIZE {cwrite[copy[0]]:.1f} KiB -> scale factors fetch "
          f"x{f_scale:.3f}, write x{w_scale:.3f}.\n")
    print(f"| kernel | FETCH_SIZE (KiB) | WRITE_SIZE (KiB) | traffic = fetch*{f_scale:.3f} + "
          f"write*{w_scale:.3f} (MiB) |")
    print("|---|---:|---:|---:|")
    table = {}
    for k in sorted(fetch):
        if "fa_" not in k:
            continue
        b = (fetch[k] * f_scale + write.get(k, 0.0) * w_scale) * 1024.0
        table[demangle_fa(k)] = int(round(b))
        print(f"| `{demangle_fa(k)}` | {fetch[k]:.1f} | {write.get(k, 0.0):.1f} | {b / 2**20:.2f} |")
    print("\n```json")
    print(json.dumps({"traffic_bytes_per_launch": table}))
    print("```")


def trace_summary(dirs):
    """Per-kernel launch statistics of rocprofv3 --kernel-trace --stats
    output directories (`*_kernel_stats.csv`, one directory per run) for
    the fa:: kernels: calls, average / min / max duration and share of the
    run's GPU time, as a markdown table per directory.  Durations of a
    --profile-config run are those of back-to-back training-step launches
    without a pre-warm, i.e. with the clocks still ramping."""
    import csv
    import glob
    for dr in dirs:
        rows = []
        for path in glob.glob(os.path.join(dr, "**", "*kernel_stats.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                rows.append(r)
        print(f"{dr}:\n")
        print("| kernel | calls | avg (us) | min (us) | max (us) | % of GPU time |")
        print("|---|---:|---:|---:|---:|---:|")
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
            print(f"| `{demangle_fa(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                  f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                  f"{float(r['Percentage']):.2f} |")
        print()
        # the training step's launches: every run of consecutive fwd ->
        # pre-pass -> fused (or fwd -> dQ -> dK/dV) dispatches, per kernel,
        # and the last 20 such sequences (the benchmark's clean in-step loop
        # runs last)
        disp = []
        for path in glob.glob(os.path.join(dr, "**", "*kernel_trace.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                disp.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                             demangle_fa(r["Kernel_Name"])))
        disp.sort()
        prefixes = (("fwd", "fa_fwd_kernel"), ("pre", "fa_bwd_preprocess_kernel"),
                    ("fused", "fa_bwd_fused_kernel"), ("dq", "fa_bwd_dq_kernel"),
                    ("dkdv", "fa_bwd_dkdv_kernel"))
        kind = [next((k for k, p in prefixes if n.startswith(p)), "") for _, _, n in disp]
        for order, title in ((("fwd", "pre", "fused"), "fwd -> pre-pass -> fused dK/dV + dQ"),
                             (("fwd", "dq", "dkdv"), "fwd -> dQ -> dK/dV")):
            seqs = [i for i in range(len(disp) - 2) if tuple(kind[i:i + 3]) == order]
            if not seqs:
                continue
            print(f"| kernel (in-step launches: {title} sequences) | launches | mean (us) | "
                  "median (us) | mean of the last 20 (us) |")
            print("|---|---:|---:|---:|---:|")
            for j, name in enumerate(order):
                d = [(disp[i + j][1] - disp[i + j][0]) / 1e3 for i in seqs]
                print(f"| {name} (`{disp[seqs[-1] + j][2]}`) | {len(d)} | {statistics.mean(d):.2f} | "
                      f"{statistics.median(d):.2f} | {statistics.mean(d[-20:]):.2f} |")
            print()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--prewarm-seconds", type=float, default=0.5,
                    help="untimed steps run for this long before the W + K measurement, "
                         "so the GPU's clocks have ramped (0 disables)")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the benchmark line, time every BASELINE config (GPU "
                         "fwd and fwd+bwd, plus the CPU baseline unless --no-cpu) and print "
                         "a table")
    ap.add_argument("--large", action="store_true",
                    help="instead of the benchmark line, time the forward and backward calls "
                         "on grids several rounds of workgroups deep and print a table")
    ap.add_argument("--rope", action="store_true",
                    help="instead of the benchmark line, time the fused QK-norm + rotary "
                         "prologue against transformers' eager one and print a table")
    ap.add_argument("--decode", action="store_true",
                    help="instead of the benchmark line, time decode-step attention "
                         "(split-KV against the unsplit kernel) and print a table")
    ap.add_argument("--llama", action="store_true",
                    help="config 5: one 16-layer Llama training step (fwd+bwd of the LM loss), "
                         "attention routed by patch_hf vs PyTorch's SDPA")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run 10 plain device copies of MIB MiB "
                         "(a kernel of known HBM traffic, to scale rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE readings) and exit")
    ap.add_argument("--profile-config", metavar="NAME",
                    help="instead of the benchmark, run the training step's kernels for one "
                         "BASELINE config (C1 ... C5-layer) --warmup + --steps times, e.g. under "
                         "rocprofv3 --pmc")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc output directories (one per counter pass) "
                         "into per-kernel counter figures and exit (no GPU needed)")
    ap.add_argument("--profile-prewarm", type=float, default=0.0, metavar="SECONDS",
                    help="with --profile-config: run the same rounds this long first")
    ap.add_argument("--traffic-summary", nargs=4,
                    metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="summarise four rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE over the "
                         "benchmark, then over --copy-calibration) into HBM bytes per launch and "
                         "exit (no GPU needed)")
    ap.add_argument("--trace-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --kernel-trace --stats output directories into "
                         "per-kernel launch tables and exit (no GPU needed)")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.traffic_summary:
        traffic_summary(args.traffic_summary)
        return
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this build has no multi-GPU path (attention would shard by heads, one GPU per "
              "process, with the kernels unchanged on each GPU's (B, S, H/g, D) share).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20)
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 10 x {n} bytes read + {n} bytes written")
        return
    if args.profile_config:
        torch.cuda.set_device(0)
        run_profile_config(args.profile_config, args.steps, args.warmup, args.profile_prewarm)
        return
    if args.configs:
        torch.cuda.set_device(0)
        run_configs(args.steps, args.warmup, not args.no_cpu, args.prewarm_seconds)
        return
    if args.decode:
        torch.cuda.set_device(0)
        run_decode(args.steps, args.warmup)
        return
    if args.large:
        torch.cuda.set_device(0)
        run_large(args.steps, args.warmup, args.prewarm_seconds)
        return
    if args.llama:
        torch.cuda.set_device(0)
        run_llama(min(args.steps, 5), min(args.warmup, 2))
        return
    if args.rope:
        torch.cuda.set_device(0)
        run_rope(args.steps, args.warmup)
        return
    from flash_attn_volta import flash_attn, flash_attn_forward
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v, do = make_inputs(dev)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))

    def fwd_bwd():
        qg.grad = kg.grad = vg.grad = None
        out = flash_attn(qg, kg, vg, causal=CAUSAL)
        out.backward(do)

    def fwd():
        flash_attn_forward(q, k, v, causal=CAUSAL)

    log(f"[bench] device={torch.cuda.get_device_name(0)} workload=(1,4096,16,64) causal fp16")
    # the same measurement first with the GPU just out of idle (reported as
    # `cold`), then after the pre-warm (`value`)
    wall_c, ev_c = time_loop(fwd_bwd, args.steps, args.warmup)
    log(f"[bench] fwd+bwd cold {ev_c * 1e3:.3f} ms/step (events), {wall_c * 1e3:.3f} ms (wall)")
    n_pre = prewarm(fwd_bwd, args.prewarm_seconds)
    log(f"[bench] pre-warm: {n_pre} steps in {args.prewarm_seconds:.2f} s")
    wall_fb, ev_fb = time_loop(fwd_bwd, args.steps, args.warmup)
    log(f"[bench] fwd+bwd {ev_fb * 1e3:.3f} ms/step (events), {wall_fb * 1e3:.3f} ms (wall)")
    prewarm(fwd, args.prewarm_seconds)
    wall_f, ev_f = time_loop(fwd, args.steps, args.warmup)
    log(f"[bench] fwd {ev_f * 1e3:.3f} ms/step (events), {wall_f * 1e3:.3f} ms (wall)")
    # the same step captured once into a HIP graph and replayed (reported
    # beside `value`, which stays the eager autograd step)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fwd_bwd()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    qg.grad = kg.grad = vg.grad = None
    with torch.cuda.graph(graph):
        flash_attn(qg, kg, vg, causal=CAUSAL).backward(do)
    prewarm(graph.replay, args.prewarm_seconds)
    wall_g, ev_g = time_loop(graph.replay, args.steps, args.warmup)
    del graph
    log(f"[bench] fwd+bwd graph replay {ev_g * 1e3:.3f} ms/step (events), {wall_g * 1e3:.3f} ms (wall)")
    kt = kernel_times(q, k, v, do, args.steps, args.warmup, args.prewarm_seconds)
    for name, r in kt.items():
        log(f"[bench] kernel {name:15s} {r['avg_us']:9.2f} us  {r['tflops']:8.1f} TFLOP/s  {r['gbs']:8.1f} GB/s")

    flops_f = fwd_flops(B, S, H, D)
    t_step = max(wall_fb, ev_fb)
    t_fwd = max(wall_f, ev_f)
    value = 5.0 * flops_f / t_step / 1e12
    fwd_tf = flops_f / t_fwd / 1e12

    # the training step launches fwd, then fa_bwd = the pre-pass and the
    # fused launch (causal D <= 64), or dQ (which also computes delta) and
    # dK/dV
    step_kernels = (("bwd_fused", "bwd_preprocess", "fwd") if FUSED_BWD
                    else ("bwd_dkdv", "bwd_dq", "fwd"))
    dom = max(step_kernels, key=lambda n: kt[n]["avg_us_in_step"])
    d = kt[dom]
    traffic, traffic_src, sym = profiled_traffic(d["kernel"])
    useful = useful_fraction(S, CAUSAL)
    t_in = d["avg_us_in_step"] * 1e-6
    achieved = d["flops"] / t_in / 1e12
    counters, counters_src = profiled_counters(sym)
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
                "frac_useful": round(useful * achieved / PEAK_FP16_TFLOPS, 4),
                "traffic": traffic, "traffic_source": traffic_src,
                "algorithmic_bytes": d["bytes"],
                "kernel": sym, "avg_us": round(d["avg_us_in_step"], 3),
                "avg_us_in_step": round(d["avg_us_in_step"], 3),
                "avg_us_in_step_evented": round(d["avg_us_in_step_evented"], 3),
                "step_us_clean": round(d["step_us_clean"], 3),
                "event_gap_us": round(d["event_gap_us"], 3),
                "avg_us_standalone": round(d["avg_us"], 3),
                "frac_standalone": round(d["tflops"] / PEAK_FP16_TFLOPS, 4),
                "flops_per_launch": d["flops"],
                "mfma_busy_counter": counters.get("mfma_busy") if counters else None,
                "counters_source": counters_src}
    if dom in MINIMAL_GEMMS:
        roofline["frac_minimal"] = round(
            minimal_flops(B, S, H, D, CAUSAL, dom) / t_in / 1e12 / PEAK_FP16_TFLOPS, 4)
        roofline["minimal_gemms"] = MINIMAL_GEMMS[dom]
    all_kernels = {}
    for n, r in kt.items():
        sym_n = profiled_traffic(r["kernel"])[2]
        row = {"kernel": sym_n, "avg_us": round(r["avg_us"], 3),
               "tflops": round(r["tflops"], 2), "frac_mfma": round(r["tflops"] / PEAK_FP16_TFLOPS, 4),
               "gbs": round(r["gbs"], 1), "frac_hbm": round(r["gbs"] / PEAK_HBM_GBS, 4)}
        if "avg_us_in_step" in r:
            tf = r["flops"] / (r["avg_us_in_step"] * 1e-6) / 1e12
            row.update({"avg_us_in_step": round(r["avg_us_in_step"], 3),
                        "frac_mfma_in_step": round(tf / PEAK_FP16_TFLOPS, 4),
                        "frac_useful_in_step": round(useful * tf / PEAK_FP16_TFLOPS, 4)})
            if n in MINIMAL_GEMMS:
                mf = minimal_flops(B, S, H, D, CAUSAL, n)
                row["frac_minimal_in_step"] = round(
                    mf / (r["avg_us_in_step"] * 1e-6) / 1e12 / PEAK_FP16_TFLOPS, 4)
            c, _ = profiled_counters(sym_n)
            if c:
                row["mfma_busy_counter"] = c.get("mfma_busy")
        all_kernels[n] = row

    cpu = None
    if not args.no_cpu:
        log("[bench] timing the CPU baseline (fp32 eager attention, fwd+bwd) ...")
        cpu = cpu_baseline()
        log(f"[bench] cpu baseline {cpu['value']:.4f} TFLOP/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REF_FWD_BWD_TFLOPS, 3),
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "flash_attn fwd+bwd step (autograd), (B,S,H,D)=(1,4096,16,64) causal",
                   "B": B, "S": S, "H": H, "D": D, "causal": CAUSAL, "sm_scale": 1.0 / math.sqrt(D),
                   "flops_convention": "fwd 4*B*H*S^2*D dense-counted, fwd+bwd 5x"},
        "pct_peak": round(100.0 * value / PEAK_FP16_TFLOPS, 2),
        "frac_minimal": round(minimal_flops(B, S, H, D, CAUSAL, "step") / t_step / 1e12
                              / PEAK_FP16_TFLOPS, 4),
        "frac_minimal_note": "share of the dense MFMA peak spent on the minimal algorithm's "
                             "work: 2 forward + 5 backward GEMMs of 2*B*H*S^2*D, causal half",
        "fwd": {"value": round(fwd_tf, 3), "unit": "TFLOP/s", "ms": round(t_fwd * 1e3, 4),
                "pct_peak": round(100.0 * fwd_tf / PEAK_FP16_TFLOPS, 2),
                "vs_baseline": round(fwd_tf / REF_FWD_TFLOPS, 3),
                "causal_useful_tflops": round(causal_useful_fwd_flops(B, S, H, D) / t_fwd / 1e12, 3)},
        "baseline": {"fwd_bwd": REF_FWD_BWD_TFLOPS, "fwd": REF_FWD_TFLOPS,
                     "hardware": "V100-SXM2-32GB (reference's published numbers)"},
        "cold": {"value": round(5.0 * flops_f / max(wall_c, ev_c) / 1e12, 3), "unit": "TFLOP/s",
                 "ms_per_step": round(max(wall_c, ev_c) * 1e3, 4),
                 "note": "the same W + K measurement as the process's first GPU work, "
                         "before the pre-warm (clocks still ramping)"},
        "prewarm_s": args.prewarm_seconds,
        "fwd_bwd_graph_replay": {"value": round(5.0 * flops_f / max(wall_g, ev_g) / 1e12, 3),
                                 "unit": "TFLOP/s", "ms": round(max(wall_g, ev_g) * 1e3, 4),
                                 "note": "same step captured once into a HIP graph and replayed"},
        "roofline": roofline,
        "kernels": all_kernels,
        "step_launches": (["fa_fwd_kernel", "fa_bwd_preprocess_kernel",
                           "fa_bwd_fused_kernel (every dK/dV block, then every dQ block)"]
                          if FUSED_BWD else
                          ["fa_fwd_kernel", "fa_bwd_dq_kernel (also computes delta)",
                           "fa_bwd_dkdv_kernel"]),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
