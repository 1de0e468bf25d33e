"""Forward attention over (B, S, H, D) fp16 tensors on an MI355X.

Drop-in for the reference's ``flash_attn_forward`` / ``flash_attn_volta``
(flash_attn_volta/triton_fa.py:291-401): same signature, defaults, return
arity, layouts and the +inf LSE rule for rows that see no key
(triton_fa.py:152-157).  The work is one launch of the hand-written gfx950
kernel behind ``fa_fwd`` (include/fa_mi355x.h); the (B, S, H, D) strides go
straight to the kernel, so there are no permute copies, and D = 32 / 64 / 128
run natively with no padding.  D = 16, which the reference also accepts
(triton_fa.py:317), is zero-padded to 32 here (an on-device copy; the padded
columns contribute exactly zero to every dot product).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _capi, _runtime
from ._runtime import VP

SUPPORTED_HEAD_DIMS = (16, 32, 64, 128)
NATIVE_HEAD_DIMS = (32, 64, 128)


class FlashAttnArgumentError(AssertionError, ValueError):
    """Invalid arguments.  Subclasses AssertionError, which is what the
    reference raises for the same checks (triton_fa.py:313-317), and
    ValueError."""


def _require(cond: bool, msg) -> None:
    """Raise FlashAttnArgumentError(msg) unless `cond`.  `msg` is a string,
    or a callable returning one: messages that format tensor shapes are
    passed as lambdas so that a passing check costs no string formatting
    (a few microseconds per call on the launch path)."""
    if not cond:
        raise FlashAttnArgumentError(msg() if callable(msg) else msg)


def _layout_ready(t: torch.Tensor) -> bool:
    """The kernels read `t`'s layout in place: unit D stride, every other
    stride (of a dim longer than 1) a non-negative multiple of 8 elements."""
    if t.stride(3) != 1:
        return False
    for dim in range(3):
        if t.size(dim) != 1 and (t.stride(dim) % 8 != 0 or t.stride(dim) < 0):
            return False
    return True


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` if the kernel can read it in place (a ready layout and a
    16-byte aligned base), else a contiguous, aligned copy."""
    if t.data_ptr() % 16 == 0 and (t.is_contiguous() or _layout_ready(t)):
        return t            # contiguous: D is a multiple of 8, so every stride is too
    return t.clone(memory_format=torch.contiguous_format)


_STRIDES = {}


def _strides_c(shape, strides):
    """C int64[4] of a (B, S, H, D) layout, 0 for size-1 dims (their stride
    is never used).  Cached per layout: the arrays are read-only."""
    key = (shape, strides)
    arr = _STRIDES.get(key)
    if arr is None:
        st = [0 if shape[i] == 1 and i < 3 else int(strides[i]) for i in range(4)]
        arr = (ctypes.c_int64 * 4)(*st)
        if len(_STRIDES) > 4096:
            _STRIDES.clear()
        _STRIDES[key] = arr
    return arr


def kernel_strides(t: torch.Tensor):
    """C int64[4] strides of tensor `t` (see _strides_c)."""
    return _strides_c(tuple(t.shape), t.stride())


def _contiguous_strides(shape) -> tuple:
    st, acc = [], 1
    for n in reversed(shape):
        st.append(acc)
        acc *= n
    return tuple(reversed(st))


def _stream_ptr(device: torch.device) -> int:
    """hipStream_t of the device's current stream."""
    return _runtime.stream_ptr(device.index)


def _on_device(device: torch.device) -> _runtime.on_device:
    """Context manager making `device` current for a launch."""
    return _runtime.on_device(device.index)


def _pad_d(t: torch.Tensor, d_to: int) -> torch.Tensor:
    return torch.nn.functional.pad(t, (0, d_to - t.size(-1)))


def flash_attn_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float | None = None,
    return_softmax_lse: bool = False,
):
    """FlashAttention forward: fp16 in/out, fp32 accumulation.

    Args:
        q, k, v: (B, N, H, D) fp16 on the GPU. D in {16, 32, 64, 128}.
        causal: apply the lower-triangular mask.
        sm_scale: softmax scale (default 1/sqrt(D)).
        return_softmax_lse: also return the per-row natural-log LSE.

    Returns:
        out (B, N, H, D) fp16 contiguous, and, if ``return_softmax_lse``,
        lse (B, H, N) fp32 contiguous (+inf for a row that sees no key).
    """
    out, lse, _ = forward_planned(q, k, v, causal, sm_scale, return_softmax_lse, False)
    return (out, lse) if return_softmax_lse else out


def _validate_fwd(q, k, v):
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "tensors must be on CUDA")
    _require(q.dtype == torch.float16 == k.dtype == v.dtype, "fp16 only")
    _require(q.shape == k.shape == v.shape, lambda: f"qkv shape mismatch {q.shape} {k.shape} {v.shape}")
    _require(q.dim() == 4, lambda: f"expected (B, N, H, D) tensors, got {tuple(q.shape)}")
    _require(q.device == k.device == v.device, "q, k, v must be on one device")
    _require(q.shape[3] in SUPPORTED_HEAD_DIMS,
             lambda: f"unsupported head_dim {q.shape[3]} (allowed: 16,32,64,128)")


def _validate_fwd_gqa(q, k, v):
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "tensors must be on CUDA")
    _require(q.dtype in _DTYPES and q.dtype == k.dtype == v.dtype,
             f"fp16 or bf16 only, all alike (got {q.dtype}, {k.dtype}, {v.dtype})")
    _require(q.device == k.device == v.device, "q, k, v must be on one device")
    _check_gqa(q, k, v)
    _require(q.shape[3] in SUPPORTED_HEAD_DIMS,
             lambda: f"unsupported head_dim {q.shape[3]} (allowed: 16,32,64,128)")


# Launch plans by call signature: everything the checks and the plan depend
# on (shapes, strides, dtypes, devices, causal, scale, LSE wanted, entry
# family), so a signature seen before skips both.  _GENERIC marks a
# signature that passed the checks but takes the general path (padded D,
# copied layouts, empty tensors).
_FWD_PLANS: dict = {}
_GENERIC = object()
_MAX_PLANS = 1024


def fwd_plan(q, k, v, causal, sm_scale, want_lse, gqa):
    """The launch plan of this call signature (a _FwdPlan, or _GENERIC for
    the general path), built after the argument checks, which raise, the
    first time the signature is seen."""
    key = (q.shape, k.shape, v.shape, q.stride(), k.stride(), v.stride(), q.dtype, k.dtype,
           v.dtype, q.device, k.device, v.device, causal, sm_scale, want_lse, gqa)
    try:
        plan = _FWD_PLANS.get(key)
    except TypeError:           # an unhashable causal / sm_scale: no caching
        key = plan = None
    if plan is None:
        (_validate_fwd_gqa if gqa else _validate_fwd)(q, k, v)
        plan = _FwdPlan.build(q, k, v, causal, sm_scale, want_lse, gqa) or _GENERIC
        if key is not None:
            if len(_FWD_PLANS) >= _MAX_PLANS:
                _FWD_PLANS.clear()
            _FWD_PLANS[key] = plan
    return plan


def forward_planned(q, k, v, causal, sm_scale, want_lse, gqa):
    """(out, lse or None, plan or None): the forward through the launch
    plan of this call signature; plan is None when the general path ran."""
    plan = fwd_plan(q, k, v, causal, sm_scale, want_lse, gqa)
    if plan is not _GENERIC:
        r = plan(q, k, v)
        if r is not None:
            return r[0], r[1], plan
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[3])
    out, lse = _forward(q, k, v, causal, sm_scale, want_lse, gqa)
    return out, lse, None


class _FwdPlan:
    """Launch plan of one forward call signature whose tensors the kernels
    read in place (native head_dim, ready layouts, nothing empty): the C
    entry point and its size / stride / scale / flag arguments, converted
    once.  A call allocates out (and LSE) and passes the data pointers and
    the current stream; the general path (_forward) gives the same
    results."""
    __slots__ = ("fn", "name", "args", "out_shape", "lse_shape", "dtype", "device", "idx",
                 "like", "ws_bytes", "causal", "sm_scale", "gqa", "sizes", "st", "q_stride",
                 "k_stride", "bwd", "cpp")

    @classmethod
    def build(cls, q, k, v, causal, sm_scale, want_lse, gqa):
        B, Sq, H, D = q.shape
        Sk, Hk = k.shape[1], k.shape[2]
        if (D not in NATIVE_HEAD_DIMS or q.numel() == 0 or Sk == 0
                or not (_layout_ready(q) and _layout_ready(k) and _layout_ready(v))):
            return None
        p = cls()
        p.causal = bool(causal)
        p.sm_scale = float(1.0 / math.sqrt(D) if sm_scale is None else sm_scale)
        p.gqa = gqa
        p.dtype, p.device, p.idx = q.dtype, q.device, q.device.index
        p.out_shape = (B, Sq, H, D)
        p.lse_shape = (B, H, Sq) if want_lse else None
        o_st = _contiguous_strides(p.out_shape)
        p.like = q.stride() == o_st          # empty_like(q) is then contiguous
        st = (kernel_strides(q), kernel_strides(k), kernel_strides(v), _strides_c(p.out_shape, o_st))
        p.sizes, p.st, p.q_stride, p.k_stride = (B, Sq, Sk, H, Hk, D), st, q.stride(), k.stride()
        p.bwd = None
        p.cpp = 0
        dt = _DTYPES[q.dtype]
        # the schedule with a workspace (split-KV for decode shapes, the
        # balanced causal one for square one-round causal grids), if any
        p.ws_bytes = int(_capi.load().fa_fwd_workspace_bytes(B, Sq, Sk, H, Hk, D, int(p.causal)))
        if p.ws_bytes:
            p.name = "fa_fwd_ws"
            p.args = _runtime.convert(p.name, 6, (p.ws_bytes, B, Sq, Sk, H, Hk, D, *st,
                                                  p.sm_scale, int(p.causal), dt))
        elif gqa:
            p.name = "fa_fwd_gqa"
            p.args = _runtime.convert(p.name, 5, (B, Sq, Sk, H, Hk, D, *st, p.sm_scale,
                                                  int(p.causal), dt))
        else:
            p.name = "fa_fwd"
            p.args = _runtime.convert(p.name, 5, (B, Sq, H, D, *st, p.sm_scale, int(p.causal)))
        p.fn = _runtime.entry(p.name)
        return p

    def __call__(self, q, k, v):
        """(out, lse) of this signature's q, k, v; None when a data pointer
        is not 16-byte aligned (the general path copies those)."""
        qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
        if (qp | kp | vp) & 15:
            return None
        out = (torch.empty_like(q) if self.like
               else torch.empty(self.out_shape, dtype=self.dtype, device=self.device))
        lse = (torch.empty(self.lse_shape, dtype=torch.float32, device=self.device)
               if self.lse_shape is not None else None)
        if _runtime.current_device() == self.idx:
            rc = self._launch(qp, kp, vp, out, lse)
        else:
            with _runtime.on_device(self.idx):
                rc = self._launch(qp, kp, vp, out, lse)
        if rc:
            _capi.check(rc, self.name)
        return out, lse

    def make_bwd(self):
        """The backward plan paired with this forward (autograd.py): its
        q, k, v are this plan's, out and dO contiguous."""
        from .backward import _BwdPlan
        q, k, v, o = self.st
        self.bwd = _BwdPlan(*self.sizes, (o, q, k, v, o), self.q_stride, self.k_stride, self.dtype,
                            self.device, self.causal, self.sm_scale, self.gqa)
        return self.bwd

    def make_cpp(self, ext):
        """Register this plan with the C++ autograd node (module `ext`,
        _fa_torch) and return its handle: sizes, flags, the q / k / v / out
        strides, contiguous dQ and dK strides, and the workspace sizes."""
        B, Sq, Sk, H, Hk, D = self.sizes
        lib = _capi.load()
        dq_st = _strides_c((B, Sq, H, D), _contiguous_strides((B, Sq, H, D)))
        dk_st = _strides_c((B, Sk, Hk, D), _contiguous_strides((B, Sk, Hk, D)))
        ints = [B, Sq, Sk, H, Hk, D, int(self.gqa), int(self.causal), _DTYPES[self.dtype]]
        for arr in (*self.st, dq_st, dk_st):
            ints += list(arr)
        ints += [self.ws_bytes,
                 int(lib.fa_bwd_gqa_workspace_bytes(B, Sq, Sk, H, Hk, D, int(self.causal))),
                 int(lib.fa_bwd_workspace_bytes(B, Sq, H, D))]
        self.cpp = ext.make_plan(ints, self.sm_scale)
        return self.cpp

    def _launch(self, qp, kp, vp, out, lse):
        stream = _runtime.stream_ptr(self.idx)
        lp = VP(lse.data_ptr()) if lse is not None else None
        if self.ws_bytes:
            ws = _runtime.workspace(self.ws_bytes, self.device, stream)
            return self.fn(VP(qp), VP(kp), VP(vp), VP(out.data_ptr()), lp, VP(ws.data_ptr()),
                           *self.args, VP(stream))
        return self.fn(VP(qp), VP(kp), VP(vp), VP(out.data_ptr()), lp, *self.args, VP(stream))


def _forward(q, k, v, causal, sm_scale, want_lse, gqa):
    """General path: pads D = 16 to 32, copies layouts the kernels cannot
    read in place, handles empty tensors.  Returns (out, lse or None)."""
    D = q.shape[-1]
    if D not in NATIVE_HEAD_DIMS:
        out, lse = _run_fwd(_pad_d(q, 32), _pad_d(k, 32), _pad_d(v, 32), causal, sm_scale,
                            want_lse, gqa)
        return out[..., :D].contiguous(), lse
    return _run_fwd(q, k, v, causal, sm_scale, want_lse, gqa)


_DTYPES = {torch.float16: _capi.FA_DTYPE_F16, torch.bfloat16: _capi.FA_DTYPE_BF16}


def _run_fwd(q, k, v, causal, sm_scale, write_lse, gqa):
    lib = _capi.load()
    B, N, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    out = torch.empty((B, N, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, N), dtype=torch.float32, device=q.device) if write_lse else None
    if out.numel() == 0 or Sk == 0:
        # no query, or no key: every row sees nothing (O = 0, LSE = +inf)
        out.zero_()
        if lse is not None:
            lse.fill_(float("inf"))
        return out, lse
    st = (kernel_strides(q), kernel_strides(k), kernel_strides(v), kernel_strides(out))
    lse_ptr = lse.data_ptr() if lse is not None else None
    with _on_device(q.device):
        stream = _stream_ptr(q.device)
        nbytes = _fwd_ws_bytes(lib, B, N, Sk, H, Hk, D, causal)
        if nbytes:
            # a schedule with a workspace: split-KV (decode) or balanced causal
            ws = _runtime.workspace(nbytes, q.device, stream)
            rc = lib.fa_fwd_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                               lse_ptr, ws.data_ptr(), nbytes, B, N, Sk, H, Hk, D, *st,
                               float(sm_scale), int(bool(causal)), _DTYPES[q.dtype], stream)
            _capi.check(rc, "fa_fwd_ws")
            return out, lse
        if gqa:
            rc = lib.fa_fwd_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse_ptr,
                                B, N, Sk, H, Hk, D, *st,
                                float(sm_scale), int(bool(causal)), _DTYPES[q.dtype], stream)
        else:
            rc = lib.fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse_ptr,
                            B, N, H, D, *st, float(sm_scale), int(bool(causal)), stream)
    _capi.check(rc, "fa_fwd_gqa" if gqa else "fa_fwd")
    return out, lse


_FWD_WS_BYTES = {}


def _fwd_ws_bytes(lib, B, Sq, Sk, H, Hk, D, causal) -> int:
    """fa_fwd_workspace_bytes for these sizes on the current device (0: the
    plain forward), cached."""
    key = (B, Sq, Sk, H, Hk, D, bool(causal), _runtime.current_device())
    nbytes = _FWD_WS_BYTES.get(key)
    if nbytes is None:
        nbytes = _FWD_WS_BYTES[key] = int(lib.fa_fwd_workspace_bytes(B, Sq, Sk, H, Hk, D,
                                                                     int(bool(causal))))
    return nbytes


def _check_gqa(q, k, v):
    """Shape rules of the grouped-query entry points: q (B, Sq, H, D),
    k and v (B, Sk, Hk, D) with H a multiple of Hk."""
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4,
             f"expected 4-D (B, N, H, D) tensors, got {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    _require(k.shape == v.shape, lambda: f"k and v shapes differ: {tuple(k.shape)} {tuple(v.shape)}")
    _require(q.shape[0] == k.shape[0], lambda: f"batch mismatch {q.shape[0]} vs {k.shape[0]}")
    _require(q.shape[3] == k.shape[3], lambda: f"head_dim mismatch {q.shape[3]} vs {k.shape[3]}")
    H, Hk = q.shape[2], k.shape[2]
    _require(Hk > 0 and H % Hk == 0,
             f"query heads ({H}) must be a multiple of key/value heads ({Hk})")


def flash_attn_forward_gqa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sm_scale: float | None = None,
    return_softmax_lse: bool = False,
):
    """Grouped-query / multi-query attention forward with independent query
    and key lengths (no counterpart in the reference; it removes the
    repeat_kv copy and the KV-cache fallback of the reference's HF patch,
    flash_attn_volta/patch_hf.py:145-162, 186-188).

    Args:
        q: (B, Sq, H, D) on the GPU; k, v: (B, Sk, Hk, D) with H a multiple
            of Hk.  Query head h uses key/value head h // (H // Hk), the head
            order of HuggingFace's ``repeat_kv``.  fp16 or bf16 (all three
            alike; the output has the same dtype, accumulation is fp32).
        causal: bottom-right aligned mask: query i sees key j iff
            j <= i + Sk - Sq (a query with no visible key gets 0 output and
            +inf LSE).  With Sq == Sk it is the usual causal mask.
        sm_scale, return_softmax_lse: as in ``flash_attn_forward``.
    """
    out, lse, _ = forward_planned(q, k, v, causal, sm_scale, return_softmax_lse, True)
    return (out, lse) if return_softmax_lse else out


# Public alias (reference: triton_fa.py:401)
flash_attn_volta = flash_attn_forward
