"""patch_hf on the CPU: patch/unpatch bookkeeping, family dispatch, the
linear-attention refusal, the causal-only mask rule and every fast-path
fallback decision, on tiny random-init transformers models (no downloads).

On the CPU the routed attention always falls back (the kernel needs the
GPU), so a patched model must reproduce the unpatched outputs bit for bit;
the GPU side (tests/test_patch_hf_gpu.py) checks the fast path numerically.
"""
from __future__ import annotations

import pytest
import torch

import hf_models
from flash_attn_volta import patch_hf


def _attn_modules(model, names):
    return [m for m in model.modules() if type(m).__name__ in names]


@pytest.mark.parametrize("family,make,names,patch,unpatch", [
    ("llama", hf_models.tiny_llama, patch_hf._LLAMA_NAMES, patch_hf.patch_llama, patch_hf.unpatch_llama),
    ("qwen2", hf_models.tiny_qwen2, patch_hf._QWEN2_NAMES, patch_hf.patch_qwen2, patch_hf.unpatch_qwen2),
    ("qwen3", hf_models.tiny_qwen3, patch_hf._QWEN3_NAMES, patch_hf.patch_qwen3, patch_hf.unpatch_qwen3),
    ("gpt2", hf_models.tiny_gpt2, patch_hf._GPT2_NAMES, patch_hf.patch_gpt2, patch_hf.unpatch_gpt2),
])
def test_patch_unpatch_and_cpu_fallback_is_exact(family, make, names, patch, unpatch):
    model = make()
    ids = hf_models.token_ids(24)
    with torch.no_grad():
        ref = model(ids).logits
    assert patch(model) == 2
    mods = _attn_modules(model, names)
    assert all(m.config._attn_implementation == patch_hf.ATTN_IMPLEMENTATION for m in mods)
    assert all(hasattr(m, "_orig_forward") for m in mods)
    # the model-level config (used to build masks) is untouched
    assert model.config._attn_implementation != patch_hf.ATTN_IMPLEMENTATION
    assert patch(model) == 2            # idempotent
    with torch.no_grad():
        out = model(ids).logits
    assert torch.equal(out, ref)        # CPU tensors -> original implementation
    assert unpatch(model) == 2
    assert all(m.config is model.config for m in mods)
    assert not any(hasattr(m, "_orig_forward") for m in mods)
    assert unpatch(model) == 0


@pytest.mark.parametrize("make,family", [(hf_models.tiny_llama, "llama"), (hf_models.tiny_qwen2, "qwen2"),
                                         (hf_models.tiny_qwen3, "qwen3"), (hf_models.tiny_gpt2, "gpt2")])
def test_patch_model_dispatch(make, family):
    model = make()
    assert patch_hf.patch_model(model) == (family, 2)


def test_patch_model_refuses_linear_attention():
    model = hf_models.tiny_mamba()
    with pytest.raises(RuntimeError) as e:
        patch_hf.patch_model(model)
    msg = str(e.value)
    assert "flash-attn-volta" in msg and "mamba" in msg and "softmax" in msg


def test_patch_model_unknown_family():
    with pytest.raises(ValueError):
        patch_hf.patch_model(torch.nn.Linear(4, 4))


def test_family_patchers_ignore_other_families():
    model = hf_models.tiny_llama()
    assert patch_hf.patch_qwen2(model) == 0
    assert patch_hf.patch_gpt2(model) == 0


def _float_causal(n, kv=None, neg=-1e4):
    kv = kv or n
    m = torch.zeros(1, 1, n, kv)
    m[..., torch.triu(torch.ones(n, kv, dtype=torch.bool), 1)] = neg
    return m


def test_causal_only_mask_rule():
    n = 8
    assert patch_hf._is_causal_only_mask(_float_causal(n), n)
    assert patch_hf._is_causal_only_mask(_float_causal(n, neg=torch.finfo(torch.float16).min), n)
    assert patch_hf._is_causal_only_mask(_float_causal(n, kv=12), n)       # top-left block only
    pad = _float_causal(n)
    pad[..., 0] = -1e4                                                     # left padding
    assert not patch_hf._is_causal_only_mask(pad, n)
    assert not patch_hf._is_causal_only_mask(torch.zeros(1, 1, n, n), n)  # bidirectional
    assert not patch_hf._is_causal_only_mask(_float_causal(n)[0, 0], n)   # not 4-D
    assert not patch_hf._is_causal_only_mask(_float_causal(n), n + 1)
    b = torch.tril(torch.ones(1, 1, n, n, dtype=torch.bool))
    assert patch_hf._is_causal_only_mask(b, n)
    b2 = b.clone()
    b2[..., 3, 1] = False
    assert not patch_hf._is_causal_only_mask(b2, n)
    assert not patch_hf._is_causal_only_mask(torch.ones(1, 1, n, n, dtype=torch.bool), n)


def _bottom_right_bool(q, kv):
    i = torch.arange(q)[:, None]
    j = torch.arange(kv)[None, :]
    return (j <= i + (kv - q)).expand(2, 1, q, kv).clone()


def _bottom_right_float(q, kv):
    m = torch.zeros(2, 1, q, kv)
    return m.masked_fill(~_bottom_right_bool(q, kv), torch.finfo(torch.float32).min)


def test_bottom_right_mask_rule():
    r = patch_hf._is_bottom_right_causal_mask
    assert r(_bottom_right_bool(5, 12), 5, 12) and r(_bottom_right_float(5, 12), 5, 12)
    assert r(_bottom_right_bool(7, 7), 7, 7)
    top_left = torch.ones(2, 1, 5, 12, dtype=torch.bool).tril()
    assert not r(top_left, 5, 12)
    assert not r(_bottom_right_bool(5, 12), 5, 13)
    assert not r(None, 5, 12)


class _Mod:
    is_causal = True


class _Enc:
    is_causal = False


def test_fast_path_decisions():
    f = patch_hf.fast_path_causal
    m, n = _Mod(), 16
    assert f(m, n, n, 64, None, 0.0, None, {}) is True
    assert f(m, n, n, 64, _float_causal(n), 0.0, None, {}) is True
    assert f(_Enc(), n, n, 64, None, 0.0, None, {}) is False       # non-causal module, no mask
    assert f(m, 1, n, 64, None, 0.0, None, {}) is True             # decode step: sees the cache
    assert f(m, 4, n, 64, None, 0.0, None, {}) is None             # chunk without a mask
    assert f(m, 4, n, 64, _bottom_right_bool(4, n), 0.0, None, {}) is True   # chunked prefill
    assert f(m, 4, n, 64, _bottom_right_float(4, n), 0.0, None, {}) is True
    static = _bottom_right_bool(4, n)
    static[..., -1] = False                                          # unused cache slot hidden
    assert f(m, 4, n, 64, static, 0.0, None, {}) is None
    assert f(m, 4, n, 64, _bottom_right_bool(4, n)[..., :n - 1], 0.0, None, {}) is None
    assert f(_Enc(), 1, n, 64, None, 0.0, None, {}) is None         # non-causal with a cache
    assert f(m, n, 4, 64, None, 0.0, None, {}) is None             # more queries than keys
    assert f(m, n, n, 64, None, 0.0, None, {"output_attentions": True}) is None
    assert f(m, n, n, 64, None, 0.1, None, {}) is None             # attention dropout
    assert f(m, n, n, 64, None, 0.0, 8, {}) is None                # narrow sliding window
    assert f(m, n, n, 64, None, 0.0, 4096, {}) is True             # window wider than S
    assert f(m, n, n, 96, None, 0.0, None, {}) is None             # head dim
    assert f(m, n, n, 64, torch.zeros(1, 1, n, n), 0.0, None, {}) is None
    assert f(_Enc(), n, n, 64, _float_causal(n), 0.0, None, {}) is None
    cross = _Mod()
    cross.is_cross_attention = True
    assert f(cross, n, n, 64, None, 0.0, None, {}) is None


def test_expand_kv_matches_transformers_repeat_kv():
    from transformers.models.llama.modeling_llama import repeat_kv
    x = torch.randn(2, 3, 5, 8)
    assert torch.equal(patch_hf._expand_kv(x, 4), repeat_kv(x, 4))
    assert patch_hf._expand_kv(x, 1) is x


@pytest.mark.parametrize("family,make,names,patch,unpatch", [
    ("llama", hf_models.tiny_llama, patch_hf._LLAMA_NAMES, patch_hf.patch_llama, patch_hf.unpatch_llama),
    ("qwen2", hf_models.tiny_qwen2, patch_hf._QWEN2_NAMES, patch_hf.patch_qwen2, patch_hf.unpatch_qwen2),
    ("qwen3", hf_models.tiny_qwen3, patch_hf._QWEN3_NAMES, patch_hf.patch_qwen3, patch_hf.unpatch_qwen3),
])
def test_fused_prologue_forward_is_installed_and_removed(family, make, names, patch, unpatch):
    model = make()
    assert patch(model, fuse_rope=False) == 2
    assert all("forward" not in m.__dict__ for m in _attn_modules(model, names))
    unpatch(model)
    assert patch(model) == 2                     # fused by default
    mods = _attn_modules(model, names)
    assert all(m.forward.__func__ is patch_hf._fused_forward for m in mods)
    ids = hf_models.token_ids(16)
    with torch.no_grad():                        # CPU: falls back to the module's own forward
        out = model(ids).logits
    assert unpatch(model) == 2
    assert all("forward" not in m.__dict__ for m in mods)
    with torch.no_grad():
        assert torch.equal(model(ids).logits, out)


def test_gpt2_gets_no_fused_prologue():
    model = hf_models.tiny_gpt2()
    patch_hf.patch_gpt2(model)
    assert all("forward" not in m.__dict__
               for m in _attn_modules(model, patch_hf._GPT2_NAMES))


class _FakeHidden:
    """Stands in for a GPU activation tensor in the prologue decision."""

    def __init__(self, B, S, hidden, dtype=torch.float16, cuda=True):
        self.shape = (B, S, hidden)
        self.dtype = dtype
        self.is_cuda = cuda

    def dim(self):
        return 3


def test_fused_prologue_decisions():
    qwen3 = _attn_modules(hf_models.tiny_qwen3(), patch_hf._QWEN3_NAMES)[0]
    llama = _attn_modules(hf_models.tiny_llama(), patch_hf._LLAMA_NAMES)[0]
    D3, DL = qwen3.head_dim, llama.head_dim
    B, S = 2, 7
    h = _FakeHidden(B, S, 128)
    t3 = (torch.ones(B, S, D3), torch.zeros(B, S, D3))
    args = patch_hf.fused_prologue_args(qwen3, h, t3)
    assert args is not None
    cos, sin, wq, wk, eps = args
    assert wq is qwen3.q_norm.weight and wk is qwen3.k_norm.weight
    assert eps == qwen3.q_norm.variance_epsilon
    la = patch_hf.fused_prologue_args(llama, h, (torch.ones(1, S, DL), torch.zeros(1, S, DL)))
    assert la is not None and la[2] is None and la[3] is None
    # fall back to transformers' own prologue:
    assert patch_hf.fused_prologue_args(qwen3, _FakeHidden(B, S, 128, cuda=False), t3) is None
    assert patch_hf.fused_prologue_args(qwen3, _FakeHidden(B, S, 128, torch.float32), t3) is None
    half = (torch.ones(B, S, D3 // 2), torch.zeros(B, S, D3 // 2))      # partial rotary
    assert patch_hf.fused_prologue_args(qwen3, h, half) is None
    assert patch_hf.fused_prologue_args(qwen3, h, (t3[0][:, :3], t3[1][:, :3])) is None
    assert patch_hf.fused_prologue_args(qwen3, h, (torch.ones(3, S, D3), torch.zeros(3, S, D3))) is None
    assert patch_hf.fused_prologue_args(qwen3, h, (t3[0].requires_grad_(True), t3[1])) is None
    assert patch_hf.fused_prologue_args(qwen3, h, None) is None
    other = hf_models.tiny_qwen3()
    m = _attn_modules(other, patch_hf._QWEN3_NAMES)[0]
    m.q_norm = torch.nn.LayerNorm(D3)                                   # another norm kind
    assert patch_hf.fused_prologue_args(m, h, (torch.ones(B, S, D3), torch.zeros(B, S, D3))) is None
    m2 = _attn_modules(hf_models.tiny_qwen3(), patch_hf._QWEN3_NAMES)[0]
    m2.k_norm.variance_epsilon = 1e-5                                   # eps differ
    assert patch_hf.fused_prologue_args(m2, h, (torch.ones(B, S, D3), torch.zeros(B, S, D3))) is None
