#!/usr/bin/env python3
"""Benchmark of the hot path: FlashAttention fwd and fwd+bwd on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (BASELINE.json metric): (B, S, H, D) = (1, 4096, 16, 64), causal,
fp16, synthetic N(0,1)*0.5 inputs already resident in HBM.  A step is one
``flash_attn`` forward + ``.backward(dO)`` -- the same boundary as the
reference's bench/backward.py:52-66 (autograd, delta pre-pass and all
kernels inside the timed region).  FLOPs follow the reference convention,
dense-counted even when causal: forward 4*B*H*S^2*D (bench/bench.py:69-71),
fwd+bwd 5x that (bench/backward.py:89-91).

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


def kernel_times(q, k, v, do, steps, warmup):
    """Average duration per launch of each kernel, by HIP events around
    back-to-back launches through the C ABI on torch's current stream
    (which is the stream the kernels are launched on)."""
    import torch
    from flash_attn_volta import _capi, flash_attn_forward
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    out, lse = flash_attn_forward(q, k, v, causal=CAUSAL, return_softmax_lse=True)
    delta = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
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
        _capi.check(lib.fa_bwd_preprocess(out.data_ptr(), do.data_ptr(), delta.data_ptr(), B, S, H, D,
                                          st["o"], st["do"], stream), "fa_bwd_preprocess")

    def dkdv():
        _capi.check(lib.fa_bwd_dkdv(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    lse.data_ptr(), delta.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                    B, S, H, D, st["do"], st["q"], st["k"], st["v"], st["dk"], st["dv"],
                                    scale, int(CAUSAL), stream), "fa_bwd_dkdv")

    def dqk():
        _capi.check(lib.fa_bwd_dq(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  lse.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                  B, S, H, D, st["do"], st["q"], st["k"], st["v"], st["dq"],
                                  scale, int(CAUSAL), stream), "fa_bwd_dq")

    pre()
    base = 2.0 * B * H * S * S * D          # one dense S x S x D GEMM
    io = B * S * H * D * 2                  # bytes of one fp16 (B,S,H,D) tensor
    rows = B * H * S * 4                    # bytes of one fp32 (B,H,S) vector
    cb = "true" if CAUSAL else "false"
    table = [
        # name, fn, kernel symbol prefix (the last template argument, the
        # in-workgroup split, is chosen by the launcher from the grid size),
        # algorithmic dense FLOPs per launch, algorithmic HBM bytes
        ("fwd", fwd, f"fa_fwd_kernel<_Float16, {D}, {cb}, ", 2 * base, 4 * io),
        ("bwd_preprocess", pre, f"fa_bwd_preprocess_kernel<_Float16, {D}>", 2.0 * B * H * S * D, 2 * io + rows),
        ("bwd_dkdv", dkdv, f"fa_bwd_dkdv_kernel<_Float16, {D}, {cb}, ", 4 * base, 6 * io + 2 * rows),
        ("bwd_dq", dqk, f"fa_bwd_dq_kernel<_Float16, {D}, {cb}, ", 3 * base, 5 * io + 2 * rows),
    ]
    res = {}
    for name, fn, sym, flops, nbytes in table:
        _, ev = time_loop(fn, steps, warmup)
        res[name] = {"kernel": sym, "avg_us": ev * 1e6, "flops": flops, "bytes": nbytes,
                     "tflops": flops / ev / 1e12, "gbs": nbytes / ev / 1e9}
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


def run_configs(steps, warmup, with_cpu):
    """Every BASELINE config: GPU forward and fwd+bwd (autograd) on the HIP
    kernels, and the CPU baseline (fp32 eager path, all host threads) for the
    same inputs.  One JSON line per config, then a markdown table."""
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
        _, t_f = time_loop(lambda: flash_attn_forward(q, k, v, causal=causal, sm_scale=sc), steps, warmup)

        def gpu_fb():
            qg.grad = kg.grad = vg.grad = None
            flash_attn(qg, kg, vg, causal=causal, sm_scale=sc).backward(do)
        t_fb = time_loop(gpu_fb, steps, warmup)[1] if with_bwd else None
        row = {"config": name, "shape": [b, s, h, d], "causal": causal,
               "gpu_fwd_us": round(t_f * 1e6, 2), "gpu_fwd_tflops": round(flops / t_f / 1e12, 2),
               "gpu_fwd_pct_peak": round(100 * flops / t_f / 1e12 / PEAK_FP16_TFLOPS, 2)}
        if with_bwd:
            row.update({"gpu_fwd_bwd_us": round(t_fb * 1e6, 2),
                        "gpu_fwd_bwd_tflops": round(5 * flops / t_fb / 1e12, 2),
                        "gpu_fwd_bwd_pct_peak": round(100 * 5 * flops / t_fb / 1e12 / PEAK_FP16_TFLOPS, 2)})
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
    hdr = ("| config | shape | GPU fwd us | GPU fwd TFLOP/s (% peak) | GPU fwd+bwd us | "
           "GPU fwd+bwd TFLOP/s (% peak) | CPU fwd TFLOP/s | CPU fwd+bwd TFLOP/s |")
    print(hdr)
    print("|---|---|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        fb = (f"{r['gpu_fwd_bwd_us']} | {r['gpu_fwd_bwd_tflops']} ({r['gpu_fwd_bwd_pct_peak']} %)"
              if "gpu_fwd_bwd_us" in r else "n/a | n/a")
        print(f"| {r['config']} | {tuple(r['shape'])}{' causal' if r['causal'] else ''} | "
              f"{r['gpu_fwd_us']} | {r['gpu_fwd_tflops']} ({r['gpu_fwd_pct_peak']} %) | {fb} | "
              f"{r.get('cpu_fwd_tflops', '-')} | {r.get('cpu_fwd_bwd_tflops', '-')} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the benchmark line, time every BASELINE config (GPU "
                         "fwd and fwd+bwd, plus the CPU baseline unless --no-cpu) and print "
                         "a table")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run 10 plain device copies of MIB MiB "
                         "(a kernel of known HBM traffic, to scale rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE readings) and exit")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this build has no multi-GPU path, see DESIGN.md for how it would shard.",
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
    if args.configs:
        torch.cuda.set_device(0)
        run_configs(args.steps, args.warmup, not args.no_cpu)
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
    wall_fb, ev_fb = time_loop(fwd_bwd, args.steps, args.warmup)
    log(f"[bench] fwd+bwd {ev_fb * 1e3:.3f} ms/step (events), {wall_fb * 1e3:.3f} ms (wall)")
    wall_f, ev_f = time_loop(fwd, args.steps, args.warmup)
    log(f"[bench] fwd {ev_f * 1e3:.3f} ms/step (events), {wall_f * 1e3:.3f} ms (wall)")
    kt = kernel_times(q, k, v, do, args.steps, args.warmup)
    for name, r in kt.items():
        log(f"[bench] kernel {name:15s} {r['avg_us']:9.2f} us  {r['tflops']:8.1f} TFLOP/s  {r['gbs']:8.1f} GB/s")

    flops_f = fwd_flops(B, S, H, D)
    t_step = max(wall_fb, ev_fb)
    t_fwd = max(wall_f, ev_f)
    value = 5.0 * flops_f / t_step / 1e12
    fwd_tf = flops_f / t_fwd / 1e12

    step_kernels = ("bwd_preprocess", "bwd_dkdv", "bwd_dq", "fwd")
    dom = max(step_kernels, key=lambda n: kt[n]["avg_us"])
    d = kt[dom]
    traffic, traffic_src, sym = profiled_traffic(d["kernel"])
    roofline = {"bound": "mfma", "achieved": round(d["tflops"], 2), "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(d["tflops"] / PEAK_FP16_TFLOPS, 4),
                "traffic": traffic, "traffic_source": traffic_src,
                "algorithmic_bytes": d["bytes"],
                "kernel": sym, "avg_us": round(d["avg_us"], 3),
                "flops_per_launch": d["flops"]}
    all_kernels = {n: {"kernel": profiled_traffic(r["kernel"])[2], "avg_us": round(r["avg_us"], 3),
                       "tflops": round(r["tflops"], 2), "frac_mfma": round(r["tflops"] / PEAK_FP16_TFLOPS, 4),
                       "gbs": round(r["gbs"], 1), "frac_hbm": round(r["gbs"] / PEAK_HBM_GBS, 4)}
                   for n, r in kt.items()}

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
        "fwd": {"value": round(fwd_tf, 3), "unit": "TFLOP/s", "ms": round(t_fwd * 1e3, 4),
                "pct_peak": round(100.0 * fwd_tf / PEAK_FP16_TFLOPS, 2),
                "vs_baseline": round(fwd_tf / REF_FWD_TFLOPS, 3),
                "causal_useful_tflops": round(causal_useful_fwd_flops(B, S, H, D) / t_fwd / 1e12, 3)},
        "baseline": {"fwd_bwd": REF_FWD_BWD_TFLOPS, "fwd": REF_FWD_TFLOPS,
                     "hardware": "V100-SXM2-32GB (reference's published numbers)"},
        "roofline": roofline,
        "kernels": all_kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
