"""fa_bwd_gqa_noalloc on the GPU: the allocation-free backward (its
workspace is the library's static device scratch buffer) against the
existing entry point fa_bwd_gqa, called through the C ABI on the same
inputs.

With a workspace of the same size -- min(fa_bwd_gqa_workspace_bytes,
FA_NOALLOC_SCRATCH_BYTES) -- both run the same kernels with the same split
schedule, so the gradients must be bit-identical.  Three calls in a row on
one GPU: a split causal D = 128 problem, then a smaller grouped-query bf16
one (Sq != Sk) over the scratch the first left behind, then the first again
over what the second left: stale scratch contents must not matter.
"""
from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

CASES = [
    # (B, Sq, Sk, H, Hk, D, dtype, causal)
    (1, 2048, 2048, 4, 4, 128, torch.float16, True),    # key- and query-block splits (~20 MiB)
    (2, 512, 700, 4, 2, 64, torch.bfloat16, True),       # smaller: GQA, bottom-right causal
    (1, 2048, 2048, 4, 4, 128, torch.float16, True),     # the first again, over stale scratch
]


def _inputs(B, Sq, Sk, H, Hk, D, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn((B, Sq, H, D), generator=g) * 0.5).to(dtype)
    k = (torch.randn((B, Sk, Hk, D), generator=g) * 0.5).to(dtype)
    v = (torch.randn((B, Sk, Hk, D), generator=g) * 0.5).to(dtype)
    do = torch.randn((B, Sq, H, D), generator=g).to(dtype)
    return [t.cuda() for t in (q, k, v, do)]


def _call(lib, fn_name, do, q, k, v, o, lse, causal, ws=None):
    from flash_attn_volta import _capi
    from flash_attn_volta.forward import kernel_strides
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    st = tuple(kernel_strides(t) for t in (do, q, k, v, o, dq, dk, dv))
    dtype = _capi.FA_DTYPE_F16 if q.dtype == torch.float16 else _capi.FA_DTYPE_BF16
    ptrs = (do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
    tail = (B, Sq, Sk, H, Hk, D, *st, 1.0 / math.sqrt(D), int(causal), dtype,
            torch.cuda.current_stream().cuda_stream)
    if ws is None:
        rc = lib.fa_bwd_gqa_noalloc(*ptrs, *tail)
    else:
        rc = lib.fa_bwd_gqa(*ptrs, ws.data_ptr(), ws.numel(), *tail)
    _capi.check(rc, fn_name)
    torch.cuda.synchronize()
    return dq, dk, dv


def test_noalloc_matches_fa_bwd_gqa_bitwise():
    from flash_attn_volta import _capi, flash_attn_forward_gqa
    lib = _capi.load()
    for i, (B, Sq, Sk, H, Hk, D, dtype, causal) in enumerate(CASES):
        print(f"[case] noalloc call {i}: B={B} Sq={Sq} Sk={Sk} H={H} Hk={Hk} D={D} {dtype} "
              f"causal={causal}", flush=True)
        q, k, v, do = _inputs(B, Sq, Sk, H, Hk, D, dtype, seed=10 + i)
        o, lse = flash_attn_forward_gqa(q, k, v, causal=causal, return_softmax_lse=True)
        full = lib.fa_bwd_gqa_workspace_bytes(B, Sq, Sk, H, Hk, D, int(causal))
        same = min(full, _capi.NOALLOC_SCRATCH_BYTES)
        # the existing entry point with a workspace of the same size, full of
        # stale bytes
        ws = torch.full((same,), 0xA5, dtype=torch.uint8, device="cuda")
        ref = _call(lib, "fa_bwd_gqa", do, q, k, v, o, lse, causal, ws)
        got = _call(lib, "fa_bwd_gqa_noalloc", do, q, k, v, o, lse, causal)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert torch.isfinite(a.float()).all(), name
            assert torch.equal(a, b), f"call {i}: {name} differs from fa_bwd_gqa " \
                f"(max-abs {(a.float() - b.float()).abs().max().item():.3e})"


def test_noalloc_under_graph_capture_matches_eager():
    """The callers fa_bwd_gqa_noalloc is for capture it into HIP graphs: one
    eager call on the device first (it looks up the scratch buffer's device
    address, which the header asks to happen before capture), then the call
    captured into a torch.cuda.CUDAGraph and replayed twice with unrelated
    eager work between the replays; every replay's gradients must equal the
    eager fa_bwd_gqa's bitwise (split causal D = 128 problem: the split
    counters are zeroed by a kernel, no memset is recorded)."""
    from flash_attn_volta import _capi, flash_attn_forward_gqa
    from flash_attn_volta.forward import kernel_strides
    lib = _capi.load()
    B, Sq, Sk, H, Hk, D, dtype, causal = CASES[0]
    print(f"[case] noalloc graph capture: B={B} Sq={Sq} H={H} D={D} causal={causal}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hk, D, dtype, seed=31)
    o, lse = flash_attn_forward_gqa(q, k, v, causal=causal, return_softmax_lse=True)
    full = lib.fa_bwd_gqa_workspace_bytes(B, Sq, Sk, H, Hk, D, int(causal))
    ws = torch.full((min(full, _capi.NOALLOC_SCRATCH_BYTES),), 0x5A, dtype=torch.uint8,
                    device="cuda")
    ref = _call(lib, "fa_bwd_gqa", do, q, k, v, o, lse, causal, ws)
    _call(lib, "fa_bwd_gqa_noalloc", do, q, k, v, o, lse, causal)   # the eager first call

    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    st = tuple(kernel_strides(t) for t in (do, q, k, v, o, dq, dk, dv))
    ptrs = (do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            rc = lib.fa_bwd_gqa_noalloc(*ptrs, B, Sq, Sk, H, Hk, D, *st, 1.0 / math.sqrt(D),
                                        int(causal), _capi.FA_DTYPE_F16,
                                        torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    _capi.check(rc, "fa_bwd_gqa_noalloc (captured)")
    for rep in range(2):
        for t in (dq, dk, dv):
            t.fill_(float("nan"))
        noise = torch.randn(1 << 20, device="cuda").sum()   # unrelated eager kernels
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from eager fa_bwd_gqa"
