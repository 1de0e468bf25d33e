"""The wrappers' launch plans and workspace cache against their general path.

A call signature seen before runs through a cached launch plan
(flash_attn_volta/forward.py, backward.py): pre-converted C arguments, no
repeated checks, the stream's cached workspace, and for autograd a
backward plan paired with the forward's.  The general path (layout copies,
D = 16 padding, per-call conversion) is the one the rest of the suite has
always exercised; these cases check that both give bitwise the same
results (the kernels are deterministic), that misaligned inputs leave the
plan for the general path, and that the workspace cache survives a
release and keeps streams apart.
"""
from __future__ import annotations

import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _eq(a, b):
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b)


CASES = [
    # B, Sq, Sk, H, Hk, D, causal, gqa, layout
    (4, 512, 512, 4, 4, 32, True, False, "bshd"),      # config 2
    (1, 1024, 1024, 8, 8, 128, True, False, "bshd"),   # split backward schedule
    (2, 300, 300, 3, 3, 64, False, False, "bhsd"),     # transposed (HF) views, ragged S
    (2, 200, 333, 8, 2, 64, True, True, "bshd"),       # grouped heads, Sq != Sk
    (1, 1, 700, 8, 1, 128, True, True, "bshd"),        # decode: split-KV forward
]


def _inputs(B, Sq, Sk, H, Hk, D, layout, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)

    def mk(S, h):
        if layout == "bhsd":
            return torch.randn((B, h, S, D), generator=g).half().cuda().transpose(1, 2)
        return torch.randn((B, S, h, D), generator=g).half().cuda()
    return mk(Sq, H), mk(Sk, Hk), mk(Sk, Hk), mk(Sq, H)


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}h{c[3]}/{c[4]}d{c[5]}"
                                             f"{'c' if c[6] else 'n'}{c[8]}" for c in CASES])
def test_plan_matches_general_path(case):
    from flash_attn_volta import forward as F, backward as Bw
    from flash_attn_volta import (flash_attn, flash_attn_backward, flash_attn_backward_gqa,
                                  flash_attn_forward, flash_attn_forward_gqa, flash_attn_gqa)
    B, Sq, Sk, H, Hk, D, causal, gqa, layout = case
    print(f"[case] plan {case}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hk, D, layout, seed=5)
    fwd = flash_attn_forward_gqa if gqa else flash_attn_forward
    bwd = flash_attn_backward_gqa if gqa else flash_attn_backward
    sc = D ** -0.5
    # general path
    o_g, l_g = F._forward(q, k, v, causal, sc, True, gqa)
    dq_g, dk_g, dv_g = Bw._backward(do, q, k, v, o_g, l_g, causal, sc, gqa)
    # planned path: first call builds the plan, the second one hits it
    for _ in range(2):
        o, lse = fwd(q, k, v, causal=causal, return_softmax_lse=True)
        assert _eq(o, o_g) and _eq(lse, l_g)
        assert o.is_contiguous() and lse.is_contiguous()
        dq, dk, dv = bwd(do, q, k, v, o, lse, causal=causal)
        assert _eq(dq, dq_g) and _eq(dk, dk_g) and _eq(dv, dv_g)
        assert dq.is_contiguous() and dk.is_contiguous() and dv.is_contiguous()
    # autograd: the C++ node (when built) and the Python Function with the
    # backward plan paired with the forward's
    from flash_attn_volta import autograd as A
    fn = flash_attn_gqa if gqa else flash_attn
    py_apply = A._apply_gqa if gqa else A._apply
    qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))
    for call in (lambda: fn(qg, kg, vg, causal=causal), lambda: py_apply(qg, kg, vg, causal, None)):
        for _ in range(2):
            qg.grad = kg.grad = vg.grad = None
            out = call()
            out.backward(do)
            assert _eq(out, o_g)
            # detach().clone() keeps each layout, so these strides are the ones above
            assert _eq(qg.grad, dq_g) and _eq(kg.grad, dk_g) and _eq(vg.grad, dv_g)
    if A._cpp is not None:
        node = type(fn(qg, kg, vg, causal=causal).grad_fn).__name__
        assert node == "CppFunction", node     # torch's name for a C++ Function's node
    # against the oracle as well, so a mistake both paths share cannot pass
    o_ref, _ = orc.attention_fwd_gqa(q.cpu(), k.cpu(), v.cpu(), causal, sc)
    assert (o.double().cpu() - torch.as_tensor(o_ref)).abs().max().item() < 1e-2


def test_misaligned_inputs_take_the_general_path():
    """A view starting 8 bytes into its storage is not 16-byte aligned: the
    plan declines it and the general path copies it."""
    from flash_attn_volta import flash_attn, flash_attn_backward, flash_attn_forward
    B, S, H, D = 2, 256, 4, 64
    print("[case] misaligned inputs", flush=True)
    q, k, v, do = _inputs(B, S, S, H, H, D, "bshd", seed=9)
    n = q.numel()

    def shifted(t):
        buf = torch.empty(n + 4, dtype=t.dtype, device=t.device)
        view = buf[4:].view(t.shape)
        view.copy_(t)
        assert view.data_ptr() % 16 == 8
        return view
    qs, ks, vs, dos = (shifted(t) for t in (q, k, v, do))
    for causal in (False, True):
        o_a, l_a = flash_attn_forward(q, k, v, causal=causal, return_softmax_lse=True)
        # the aligned call above made the plan for this signature
        o_b, l_b = flash_attn_forward(qs, ks, vs, causal=causal, return_softmax_lse=True)
        assert _eq(o_a, o_b) and _eq(l_a, l_b)
        g_a = flash_attn_backward(do, q, k, v, o_a, l_a, causal=causal)
        g_b = flash_attn_backward(dos, qs, ks, vs, o_b, l_b, causal=causal)
        assert all(_eq(x, y) for x, y in zip(g_a, g_b))
        qg = qs.detach().clone().requires_grad_()
        out = flash_attn(qg, ks, vs, causal=causal)
        out.backward(dos)
        assert _eq(out, o_a) and _eq(qg.grad, g_a[0])


def test_workspace_cache_release_and_streams():
    from flash_attn_volta import _runtime, flash_attn_backward, flash_attn_forward
    from flash_attn_volta import release_workspaces
    B, S, H, D = 1, 1024, 8, 128
    print("[case] workspace cache", flush=True)
    q, k, v, do = _inputs(B, S, S, H, H, D, "bshd", seed=13)
    o, lse = flash_attn_forward(q, k, v, causal=True, return_softmax_lse=True)
    ref = flash_attn_backward(do, q, k, v, o, lse, causal=True)
    assert _runtime.workspace_bytes_held() > 0
    release_workspaces()
    assert _runtime.workspace_bytes_held() == 0
    again = flash_attn_backward(do, q, k, v, o, lse, causal=True)
    assert all(_eq(x, y) for x, y in zip(ref, again))
    # a second stream gets a workspace of its own; both streams' results
    # match the first stream's
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        on_side = flash_attn_backward(do, q, k, v, o, lse, causal=True)
        for t in (do, q, k, v, o, lse):
            t.record_stream(side)
    main = flash_attn_backward(do, q, k, v, o, lse, causal=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert len({key[1] for key in _runtime._WS}) >= 2
    assert all(_eq(x, y) for x, y in zip(ref, on_side))
    assert all(_eq(x, y) for x, y in zip(ref, main))


def test_cpp_node_gradient_forms():
    """The C++ node's backward takes dO in any layout and dtype (made
    contiguous, cast to the forward's dtype), uses the split or delta-only
    workspace by split_workspace at forward time, and accumulates into
    existing .grad like any autograd node."""
    from flash_attn_volta import autograd as A
    from flash_attn_volta import backward as Bw
    from flash_attn_volta import flash_attn, flash_attn_backward, flash_attn_forward
    if A._cpp is None:
        pytest.skip("_fa_torch is not built")
    B, S, H, D = 1, 1024, 8, 128
    print("[case] C++ node gradient forms", flush=True)
    q, k, v, do = _inputs(B, S, S, H, H, D, "bshd", seed=17)
    o, lse = flash_attn_forward(q, k, v, causal=True, return_softmax_lse=True)
    ref = flash_attn_backward(do, q, k, v, o, lse, causal=True)
    qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))
    # dO transposed (non-contiguous) and in fp32
    do_t = do.float().transpose(1, 2).contiguous().transpose(1, 2)
    out = flash_attn(qg, kg, vg, causal=True)
    out.backward(do_t)
    assert _eq(qg.grad, ref[0]) and _eq(kg.grad, ref[1]) and _eq(vg.grad, ref[2])
    # a second backward accumulates
    flash_attn(qg, kg, vg, causal=True).backward(do)
    assert _eq(qg.grad, 2 * ref[0])     # x + x rounds exactly in fp16
    # delta-only workspace (the unsplit schedule): same results to rounding
    Bw.split_workspace = False
    try:
        qg.grad = kg.grad = vg.grad = None
        flash_attn(qg, kg, vg, causal=True).backward(do)
    finally:
        Bw.split_workspace = True
    for got, want in zip((qg.grad, kg.grad, vg.grad), ref):
        assert (got.float() - want.float()).abs().max().item() < 1e-2    # the suite's max-abs bar


def test_plan_cache_eviction(monkeypatch):
    """More signatures than the plan caches hold: they are cleared and
    rebuilt, and every call still matches the general path."""
    from flash_attn_volta import backward as Bw, forward as F
    from flash_attn_volta import flash_attn, flash_attn_backward, flash_attn_forward
    monkeypatch.setattr(F, "_MAX_PLANS", 4)
    monkeypatch.setattr(Bw, "_MAX_PLANS", 4)
    print("[case] plan cache eviction", flush=True)
    for rep in range(2):
        for S in (64, 96, 130, 200, 256, 300):
            q, k, v, do = _inputs(1, S, S, 2, 2, 64, "bshd", seed=S)
            o_g, l_g = F._forward(q, k, v, True, 0.125, True, False)
            o, lse = flash_attn_forward(q, k, v, causal=True, sm_scale=0.125, return_softmax_lse=True)
            assert _eq(o, o_g) and _eq(lse, l_g)
            g = flash_attn_backward(do, q, k, v, o, lse, causal=True, sm_scale=0.125)
            g_g = Bw._backward(do, q, k, v, o_g, l_g, True, 0.125, False)
            assert all(_eq(x, y) for x, y in zip(g, g_g))
            qg = q.clone().requires_grad_()
            flash_attn(qg, k, v, causal=True, sm_scale=0.125).backward(do)
            assert _eq(qg.grad, g_g[0])
        assert len(F._FWD_PLANS) <= 4 and len(Bw._BWD_PLANS) <= 4


def test_two_threads_two_streams():
    """Two host threads, each on its own stream, run autograd steps at once:
    the plan caches, the workspace cache and the C++ node are shared; every
    step's gradients equal the single-threaded ones."""
    import threading
    from flash_attn_volta import flash_attn
    print("[case] two threads", flush=True)
    shapes = [(2, 512, 4, 64), (1, 1024, 8, 128)]
    refs = []
    inputs = []
    for i, (B, S, H, D) in enumerate(shapes):
        q, k, v, do = _inputs(B, S, S, H, H, D, "bshd", seed=40 + i)
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        flash_attn(qg, kg, vg, causal=True).backward(do)
        refs.append((qg.grad.clone(), kg.grad.clone(), vg.grad.clone()))
        inputs.append((q, k, v, do))
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            q, k, v, do = inputs[i]
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(10):
                    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
                    flash_attn(qg, kg, vg, causal=True).backward(do)
                    got = (qg.grad, kg.grad, vg.grad)
                    stream.synchronize()
                    if not all(_eq(a, b) for a, b in zip(got, refs[i])):
                        errors.append(f"thread {i}: gradients differ")
                        return
        except Exception as e:       # reported below, in the test's own thread
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(shapes))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
