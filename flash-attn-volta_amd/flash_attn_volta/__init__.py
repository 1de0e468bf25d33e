"""flash_attn_volta -- FlashAttention forward + backward for AMD Instinct MI355X (gfx950).

Drop-in replacement for the reference package of the same name
(flash_attn_volta/__init__.py:1-24): the same public functions, signatures
and (B, N, H, D) fp16 layout, backed by hand-written HIP kernels in the
C-ABI library libfa_mi355x.so instead of Triton.

Public API:
    flash_attn_forward(q, k, v, causal=False, sm_scale=None,
                       return_softmax_lse=False)         -> out [, lse]
    flash_attn_volta  (alias of flash_attn_forward)
    flash_attn(q, k, v, causal=False, sm_scale=None)     -> out  (autograd-aware)
    flash_attn_backward(do, q, k, v, o, lse,
                        causal=False, sm_scale=None)     -> (dq, dk, dv)

q, k, v, out: (batch, seq, n_heads, head_dim) fp16; lse: (B, H, N) fp32.

Beyond the reference (its wrapper requires q, k, v of one shape):
    flash_attn_forward_gqa / flash_attn_backward_gqa / flash_attn_gqa
        grouped-query and multi-query attention, k and v (B, Sk, Hk, D)
        with H a multiple of Hk, Sq != Sk with a bottom-right causal
        mask (KV-cache prefill continuation), and bf16 as well as fp16.
    apply_rotary_qk / rope_qk_forward / rope_qk_backward
        the attention prologue fused into one pass: optional per-head
        RMSNorm (Qwen3's q_norm / k_norm) and rotary position embedding
        of q and k.
    flash_attn_op
        flash_attn_gqa as torch.library custom ops (flash_attn_volta::fwd,
        flash_attn_volta::bwd) with fake-tensor and autograd registrations,
        so torch.compile keeps the call as one graph node.
    release_workspaces
        free the backward / split-KV workspaces, which are cached per stream
        and reused by later calls.
"""

from .forward import flash_attn_forward, flash_attn_forward_gqa, flash_attn_volta
from .backward import flash_attn_backward, flash_attn_backward_gqa
from .autograd import flash_attn, flash_attn_gqa
from .rope import apply_rotary_qk, rope_qk_backward, rope_qk_forward
from .ops import flash_attn_op
from ._runtime import release_workspaces

__all__ = [
    "flash_attn_forward",
    "flash_attn_volta",
    "flash_attn_backward",
    "flash_attn",
    "flash_attn_forward_gqa",
    "flash_attn_backward_gqa",
    "flash_attn_gqa",
    "apply_rotary_qk",
    "rope_qk_forward",
    "rope_qk_backward",
    "flash_attn_op",
    "release_workspaces",
]
__version__ = "0.4.0"
