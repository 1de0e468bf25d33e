"""Route HuggingFace transformers attention through ``flash_attn_volta``.

Same public surface as the reference's patch module
(flash_attn_volta/patch_hf.py): ``patch_{gpt2,qwen2,qwen3,llama}(model) ->
int``, the matching ``unpatch_*``, ``patch_model(model) -> (family, n)``
with the same dispatch order (GPT-2, Qwen3, Qwen2, Llama; :409-417) and the
same loud refusal of linear-attention / state-space models (:358-407), and
``_is_causal_only_mask`` (:29-48).

The reference replaces whole attention ``forward`` methods written against
transformers 4.44.  transformers 5.x changed those signatures; every
decoder attention module now computes post-RoPE, post-cache (B, H, S, D)
query/key/value and hands them to
``ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
eager_attention_forward)``.  This module therefore registers one attention
function, ``"flash_attn_volta"``, in transformers' ``AttentionInterface``
and routes each patched module to it by giving that module a shallow copy
of its config whose ``_attn_implementation`` names it.  Unpatching restores
the module's own config object.  Projections, QK-norm, RoPE, caches and the
output projection stay HuggingFace's own code for every family.

The fast path is taken under the reference's conditions (:68-75,
:443-452): self-attention, no ``output_attentions``, no attention dropout,
no sliding window narrower than the sequence, and an attention mask that
is absent (the module is causal) or causal-only.  Two of the reference's
restrictions are lifted by the grouped-query kernels (flash_attn_gqa):
GQA/MQA key/value heads are read in place instead of being expanded with
repeat_kv (:186-188, :470-471), and a KV cache with content
(kv_len > q_len: decode steps, chunked prefill) no longer falls back
(:145-162) when its mask is the bottom-right-aligned causal mask (query i
sees cache positions j <= i + kv_len - q_len), as a dynamic cache gives.
Anything else runs the module's original attention implementation
unchanged.

For the Llama, Qwen2 and Qwen3 families the patch also replaces the
module's forward (the reference does the same for transformers 4.44,
patch_hf.py:164-198, 284-313, 425-480) so that the attention prologue --
Qwen3's q_norm / k_norm and the rotary embedding, which transformers runs as
some ten elementwise kernels per tensor and direction -- is one fused
kernel (apply_rotary_qk) that also writes q and k in the (B, S, H, D)
layout the attention kernels read.  The projections, cache update and
output projection are the module's own layers, called as transformers
calls them.  A module whose prologue is not the standard one (another norm
type, partial rotary tables, CPU tensors) runs its original forward.
``fuse_rope=False`` keeps transformers' own prologue.
"""
from __future__ import annotations

import copy
import sys
import types
from typing import Optional, Tuple

import torch

from .autograd import flash_attn, flash_attn_gqa
from .rope import ROPE_HEAD_DIMS, apply_rotary_qk

ATTN_IMPLEMENTATION = "flash_attn_volta"

_GPT2_NAMES = {"GPT2Attention"}
_QWEN2_NAMES = {"Qwen2Attention", "Qwen2SdpaAttention", "Qwen2FlashAttention2"}
_QWEN3_NAMES = {"Qwen3Attention", "Qwen3SdpaAttention", "Qwen3FlashAttention2"}
_LLAMA_NAMES = {"LlamaAttention", "LlamaSdpaAttention", "LlamaFlashAttention2"}


def _is_causal_only_mask(mask: torch.Tensor, q_len: int) -> bool:
    """True if ``mask`` (4-D, (.., q_len, kv_len >= q_len)) is the plain causal
    mask on its top-left q_len x q_len block.

    Float masks (added to scores): lower triangle incl. diagonal |m| <= 1e-3,
    strict upper triangle <= -1 (the reference's rule, patch_hf.py:29-48).
    Bool masks (transformers 5.x; True = attend): lower triangle incl.
    diagonal True, strict upper triangle False.
    """
    if mask is None or mask.dim() != 4:
        return False
    if mask.size(-2) != q_len or mask.size(-1) < q_len:
        return False
    m = mask[..., :q_len, :q_len]
    tri = torch.tril(torch.ones(q_len, q_len, device=mask.device, dtype=torch.bool))
    if m.dtype == torch.bool:
        return bool(m[..., tri].all()) and not bool(m[..., ~tri].any())
    if (m[..., tri].abs() > 1e-3).any():
        return False
    if (m[..., ~tri] > -1.0).any():
        return False
    return True


def _is_bottom_right_causal_mask(mask: torch.Tensor, q_len: int, kv_len: int) -> bool:
    """True if ``mask`` (4-D, (.., q_len, kv_len)) lets query i see exactly
    the keys j <= i + kv_len - q_len: the causal mask of q_len new tokens
    appended to a cache of kv_len - q_len.  Float masks: visible entries
    |m| <= 1e-3, hidden <= -1; bool masks: True = attend."""
    if mask is None or mask.dim() != 4:
        return False
    if mask.size(-2) != q_len or mask.size(-1) != kv_len or kv_len < q_len:
        return False
    i = torch.arange(q_len, device=mask.device)[:, None]
    j = torch.arange(kv_len, device=mask.device)[None, :]
    vis = j <= i + (kv_len - q_len)
    if mask.dtype == torch.bool:
        return bool(mask[..., vis].all()) and not bool(mask[..., ~vis].any())
    if (mask[..., vis].abs() > 1e-3).any():
        return False
    if (mask[..., ~vis] > -1.0).any():
        return False
    return True


def _original_interface(module):
    """The attention function the module would use unpatched."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    impl = getattr(module, "_fav_orig_impl", None)
    eager = getattr(sys.modules.get(type(module).__module__), "eager_attention_forward", None)
    if eager is None:
        from transformers.models.llama.modeling_llama import eager_attention_forward as eager
    if impl is None or impl == "eager":
        return eager
    return ALL_ATTENTION_FUNCTIONS.get_interface(impl, eager)


def _expand_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """(B, Hkv, S, D) -> (B, Hkv * n_rep, S, D), each kv head repeated n_rep
    times consecutively (transformers' repeat_kv)."""
    if n_rep == 1:
        return x
    B, Hkv, S, D = x.shape
    return x[:, :, None].expand(B, Hkv, n_rep, S, D).reshape(B, Hkv * n_rep, S, D)


def fast_path_causal(module, q_len: int, kv_len: int, head_dim: int,
                     attention_mask: Optional[torch.Tensor], dropout: Optional[float],
                     sliding_window: Optional[int], kwargs: dict) -> Optional[bool]:
    """Decide whether an attention call may run on the flash kernel.

    Returns None to fall back to the module's original implementation, else
    the causal flag to run the kernel with (bottom-right aligned when
    kv_len > q_len).  Fallbacks mirror the reference (patch_hf.py:68-75,
    :443-452): output_attentions, cross-attention, a head mask, a mask that
    is not causal-only; plus what the kernel does not implement here:
    attention dropout, a sliding window narrower than the sequence, head
    dims outside {16, 32, 64, 128}.  A KV cache with content (kv_len >
    q_len, where the reference always falls back, :145-162) runs on the
    kernel when the module is causal and the mask is the bottom-right
    causal mask, or absent for a single new token; a cache whose mask hides
    more (a static cache's unused tail, padding) falls back.
    """
    causal = bool(getattr(module, "is_causal", True))
    if kwargs.get("output_attentions", False):
        return None
    if getattr(module, "is_cross_attention", False) or kwargs.get("head_mask") is not None:
        return None
    if dropout not in (None, 0.0):
        return None
    if sliding_window is not None and sliding_window < kv_len:
        return None
    if head_dim not in (16, 32, 64, 128):
        return None
    if q_len != kv_len:
        if not causal or kv_len < q_len:
            return None
        if attention_mask is None:
            return True if q_len == 1 else None
        return True if _is_bottom_right_causal_mask(attention_mask, q_len, kv_len) else None
    if attention_mask is not None:
        if not (causal and _is_causal_only_mask(attention_mask, q_len)):
            return None
    return causal


def flash_attn_volta_attention(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    dropout: float = 0.0,
    scaling: Optional[float] = None,
    sliding_window: Optional[int] = None,
    **kwargs,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """transformers 5.x attention function: (B, H, S, D) in, (B, S, H, D) out."""
    causal = None
    if query.is_cuda:
        causal = fast_path_causal(module, query.shape[2], key.shape[2], query.shape[-1],
                                  attention_mask, dropout, sliding_window, kwargs)
    if causal is None:
        return _original_interface(module)(module, query, key, value, attention_mask,
                                           dropout=dropout, scaling=scaling,
                                           sliding_window=sliding_window, **kwargs)

    out_dtype = query.dtype
    # bf16 models stay in bf16 (their activations may not fit fp16); the
    # rest run in fp16 like the reference (patch_hf.py:473-475)
    kdt = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float16
    q = query.transpose(1, 2).to(kdt)
    k = key.transpose(1, 2).to(kdt)
    v = value.transpose(1, 2).to(kdt)
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    if q.shape == k.shape and kdt == torch.float16:
        out = flash_attn(q, k, v, causal=causal, sm_scale=float(scaling))
    else:
        # grouped K/V heads, a cache or bf16: read in place, no repeat_kv copy
        out = flash_attn_gqa(q, k, v, causal=causal, sm_scale=float(scaling))
    return out.to(out_dtype), None


# Norm modules that compute weight * x / sqrt(mean(x^2) + eps) over the last
# dimension (transformers' Qwen3RMSNorm and its identical siblings).
_RMSNORM_NAMES = {"Qwen3RMSNorm", "Qwen2RMSNorm", "LlamaRMSNorm"}


def _qk_norm(module, name: str, D: int):
    """(weight, eps) of the module's q_norm / k_norm; (None, None) when it
    has none; raises LookupError for a norm the fused kernel does not
    implement."""
    m = getattr(module, name, None)
    if m is None or isinstance(m, torch.nn.Identity):
        return None, None
    w = getattr(m, "weight", None)
    eps = getattr(m, "variance_epsilon", None)
    if type(m).__name__ not in _RMSNORM_NAMES or w is None or tuple(w.shape) != (D,) or eps is None:
        raise LookupError(name)
    return w, float(eps)


def fused_prologue_args(module, hidden_states: torch.Tensor, position_embeddings):
    """The arguments of apply_rotary_qk for this call, ``(cos, sin, q_norm
    weight, k_norm weight, eps)``, or None when the prologue must run as
    transformers writes it: CPU or non-16-bit activations, a head dim the
    kernel lacks, rotary tables that are not (B or 1, S, head_dim) (partial
    rotary), tables that require grad, or a QK-norm of another kind."""
    if not hidden_states.is_cuda or hidden_states.dtype not in (torch.float16, torch.bfloat16):
        return None
    D = getattr(module, "head_dim", None)
    if D not in ROPE_HEAD_DIMS or hidden_states.dim() != 3:
        return None
    if not isinstance(position_embeddings, (tuple, list)) or len(position_embeddings) != 2:
        return None
    cos, sin = position_embeddings
    if not (isinstance(cos, torch.Tensor) and isinstance(sin, torch.Tensor)):
        return None
    B, S = hidden_states.shape[:2]
    if cos.shape != sin.shape or cos.dim() != 3 or tuple(cos.shape[1:]) != (S, D) \
            or cos.shape[0] not in (1, B) or cos.requires_grad or sin.requires_grad:
        return None
    try:
        wq, eq = _qk_norm(module, "q_norm", D)
        wk, ek = _qk_norm(module, "k_norm", D)
    except LookupError:
        return None
    if eq is not None and ek is not None and eq != ek:
        return None
    eps = eq if eq is not None else (ek if ek is not None else 1e-6)
    return cos, sin, wq, wk, eps


def _fused_forward(self, hidden_states: torch.Tensor, position_embeddings=None,
                   attention_mask: Optional[torch.Tensor] = None, past_key_values=None, **kwargs):
    """transformers 5.x Llama / Qwen2 / Qwen3 attention forward with the
    q/k prologue fused (same arguments and results as the module's own)."""
    args = fused_prologue_args(self, hidden_states, position_embeddings)
    if args is None:
        return self._orig_forward(hidden_states, position_embeddings=position_embeddings,
                                  attention_mask=attention_mask, past_key_values=past_key_values,
                                  **kwargs)
    cos, sin, wq, wk, eps = args
    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    q = self.q_proj(hidden_states).view(hidden_shape)          # (B, S, H, D)
    k = self.k_proj(hidden_states).view(hidden_shape)
    v = self.v_proj(hidden_states).view(hidden_shape)
    q, k = apply_rotary_qk(q, k, cos, sin, wq, wk, eps)
    query_states, key_states, value_states = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if past_key_values is not None:
        key_states, value_states = past_key_values.update(key_states, value_states, self.layer_idx)
    if "sliding_window" in self.__dict__ or hasattr(type(self), "sliding_window"):
        kwargs.setdefault("sliding_window", self.sliding_window)
    attn_output, attn_weights = flash_attn_volta_attention(
        self, query_states, key_states, value_states, attention_mask,
        dropout=0.0 if not self.training else self.attention_dropout,
        scaling=self.scaling, **kwargs)
    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    return self.o_proj(attn_output), attn_weights


_registered = False


def _register() -> None:
    global _registered
    if _registered:
        return
    from transformers.modeling_utils import AttentionInterface
    AttentionInterface.register(ATTN_IMPLEMENTATION, flash_attn_volta_attention)
    _registered = True


def _patch(model: torch.nn.Module, names, fuse_rope: bool = False) -> int:
    _register()
    n = 0
    for mod in model.modules():
        if type(mod).__name__ not in names or not hasattr(mod, "config"):
            continue
        if not hasattr(mod, "_fav_orig_config"):
            cfg = mod.config
            mod._fav_orig_config = cfg
            mod._fav_orig_impl = getattr(cfg, "_attn_implementation", None)
            routed = copy.copy(cfg)
            # set the backing field directly: the property setter would also
            # rewrite sub-configs, which the shallow copy shares
            routed._attn_implementation_internal = ATTN_IMPLEMENTATION
            mod.config = routed
            mod._orig_forward = mod.forward
            if fuse_rope and all(hasattr(mod, a) for a in ("q_proj", "k_proj", "v_proj",
                                                           "o_proj", "head_dim")):
                mod.forward = types.MethodType(_fused_forward, mod)
        n += 1
    return n


def _unpatch(model: torch.nn.Module, names) -> int:
    n = 0
    for mod in model.modules():
        if type(mod).__name__ in names and hasattr(mod, "_fav_orig_config"):
            mod.config = mod._fav_orig_config
            del mod._fav_orig_config
            del mod._fav_orig_impl
            if "_orig_forward" in mod.__dict__:
                del mod._orig_forward
            mod.__dict__.pop("forward", None)
            n += 1
    return n


def patch_gpt2(model: torch.nn.Module) -> int:
    """Patch every GPT2Attention block on ``model``. Returns count patched."""
    return _patch(model, _GPT2_NAMES)


def unpatch_gpt2(model: torch.nn.Module) -> int:
    return _unpatch(model, _GPT2_NAMES)


def patch_qwen2(model: torch.nn.Module, fuse_rope: bool = True) -> int:
    """Patch every Qwen2 attention block on ``model``. Returns count patched.
    ``fuse_rope``: run the rotary prologue as one fused kernel."""
    return _patch(model, _QWEN2_NAMES, fuse_rope)


def unpatch_qwen2(model: torch.nn.Module) -> int:
    return _unpatch(model, _QWEN2_NAMES)


def patch_qwen3(model: torch.nn.Module, fuse_rope: bool = True) -> int:
    """Patch every Qwen3 attention block. Returns count patched; 0 when the
    installed transformers has no Qwen3.  ``fuse_rope``: run QK-norm and the
    rotary embedding as one fused kernel (else transformers' own modules,
    applied before the routed attention call)."""
    try:
        from transformers.models.qwen3 import modeling_qwen3  # noqa: F401
    except ImportError:
        return 0
    return _patch(model, _QWEN3_NAMES, fuse_rope)


def unpatch_qwen3(model: torch.nn.Module) -> int:
    return _unpatch(model, _QWEN3_NAMES)


def patch_llama(model: torch.nn.Module, fuse_rope: bool = True) -> int:
    """Patch every Llama attention block on ``model``. Returns count patched.
    ``fuse_rope``: run the rotary prologue as one fused kernel."""
    return _patch(model, _LLAMA_NAMES, fuse_rope)


def unpatch_llama(model: torch.nn.Module) -> int:
    return _unpatch(model, _LLAMA_NAMES)


def _is_qwen2_attention(mod) -> bool:
    return type(mod).__name__ in _QWEN2_NAMES


def _is_qwen3_attention(mod) -> bool:
    return type(mod).__name__ in _QWEN3_NAMES


def _is_llama_attention(mod) -> bool:
    return type(mod).__name__ in _LLAMA_NAMES


# Linear-attention / state-space families the kernel must refuse (the
# families of reference patch_hf.py:358-387): each family's marker module
# classes, tested in this order (a model holding markers of two families
# reports the first).
_LINEAR_ATTN_MARKERS = (
    ("mamba", ("MambaMixer",)),
    ("mamba2", ("Mamba2Mixer",)),
    ("rwkv", ("RwkvSelfAttention", "RwkvLinearAttention")),
    ("recurrent_gemma", ("RecurrentGemmaRecurrentBlock",)),
    ("retnet", ("RetNetAttention",)),
)


def _linear_attn_family(model: torch.nn.Module) -> Optional[str]:
    """Family name of a linear-attention or state-space model (the first
    entry of _LINEAR_ATTN_MARKERS with a marker class among the model's
    modules), else None."""
    classes = {type(model).__name__} | {type(m).__name__ for m in model.modules()}
    return next((fam for fam, markers in _LINEAR_ATTN_MARKERS if classes.intersection(markers)),
                None)


def patch_model(model: torch.nn.Module, fuse_rope: bool = True) -> Tuple[str, int]:
    """Detect the model family and patch it. Returns ``(family, n_patched)``.
    ``fuse_rope`` is passed to the Llama / Qwen2 / Qwen3 patches.

    Raises ``RuntimeError`` for linear-attention / state-space models, for
    which softmax attention would be mathematically wrong, and
    ``ValueError`` for an unknown family.
    """
    fam = _linear_attn_family(model)
    if fam is not None:
        raise RuntimeError(
            f"flash-attn-volta only supports softmax MHA / GQA — model uses {fam}. "
            "Refusing to patch a linear-attention / state-space architecture."
        )
    cls = type(model).__name__
    mods = list(model.modules())
    if "GPT2" in cls or any(type(m).__name__ in _GPT2_NAMES for m in mods):
        return "gpt2", patch_gpt2(model)
    if "Qwen3" in cls or any(_is_qwen3_attention(m) for m in mods):
        return "qwen3", patch_qwen3(model, fuse_rope)
    if "Qwen2" in cls or any(_is_qwen2_attention(m) for m in mods):
        return "qwen2", patch_qwen2(model, fuse_rope)
    if "Llama" in cls or any(_is_llama_attention(m) for m in mods):
        return "llama", patch_llama(model, fuse_rope)
    raise ValueError(f"no patch known for model class {cls}")
