"""Host-side launch machinery of the wrappers: pre-converted C-ABI calls,
the per-stream workspace cache, and the current device / stream queries.

A ctypes call through declared ``argtypes`` converts every argument on every
call, about 2 us for the 16-30 arguments of these entry points.  A launch
plan (forward.py, backward.py) converts the arguments fixed by a call
signature (sizes, strides, scale, flags) once, with ``convert``, and per
call wraps only the data pointers and the stream in ``c_void_p``;
``entry`` returns the same C function without argument conversion for
that.
"""
from __future__ import annotations

import collections
import ctypes

import torch

from . import _capi

VP = ctypes.c_void_p

_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_GET_DEVICE = getattr(torch._C, "_cuda_getDevice", None)
_CAPTURING = getattr(torch._C, "_cuda_isCurrentStreamCapturing", None)


def stream_ptr(index: int) -> int:
    """hipStream_t of device `index`'s current stream (the raw query skips
    building a Stream object; same value)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(index).cuda_stream


def current_device() -> int:
    if _GET_DEVICE is not None:
        return _GET_DEVICE()
    return torch.cuda.current_device()


def capturing() -> bool:
    """True while the current stream is being captured into a graph."""
    if _CAPTURING is not None:
        return _CAPTURING()
    return torch.cuda.is_current_stream_capturing()


class on_device:
    """Make device `index` current for the duration of a launch, skipping
    the context switch in the common case where it already is."""
    __slots__ = ("idx", "prev")

    def __init__(self, index: int):
        self.idx = index

    def __enter__(self):
        self.prev = current_device()
        if self.prev != self.idx:
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev != self.idx:
            torch.cuda.set_device(self.prev)
        return False


_raw_lib = None


def entry(name: str):
    """C function `name` of the library with no ctypes argument conversion:
    every argument must already be a ctypes object of the declared type
    (``convert``) or a ``c_void_p``.  Returns an int status."""
    global _raw_lib
    if _raw_lib is None:
        _capi.load()                    # existence and ABI checks
        _raw_lib = ctypes.CDLL(_capi.LIB_PATH)
    fn = getattr(_raw_lib, name)
    fn.restype = ctypes.c_int
    return fn


def convert(name: str, first: int, values) -> tuple:
    """ctypes objects for arguments first, first + 1, ... of C function
    `name`, by the argtypes _capi declares for it (int64[4] stride arrays
    pass as they are: an array argument passes its address)."""
    types = getattr(_capi.load(), name).argtypes[first:first + len(values)]
    if len(types) != len(values):
        raise ValueError(f"{name}: {len(values)} values for {len(types)} arguments from {first}")
    return tuple(v if isinstance(v, ctypes.Array) else t(v) for t, v in zip(types, values))


# Workspaces by (device index, stream): reused by every call on that stream
# (stream order keeps one call's use of it before the next one's), grown
# when a call needs more.  A call made while its stream is being captured
# into a graph gets a fresh tensor instead: the graph keeps the addresses it
# recorded, which a later growth here would free.  At most
# MAX_CACHED_STREAMS streams keep one (least recently used dropped first),
# so threads drawing streams from a pool cannot pin a workspace each (up to
# ~64 MiB for the split schedule of a small causal grid); the memory of a
# dropped one goes back to torch's caching allocator.
MAX_CACHED_STREAMS = 4
_WS: "collections.OrderedDict" = collections.OrderedDict()


def workspace(nbytes: int, device: torch.device, stream: int) -> torch.Tensor:
    if capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        _WS.pop(key, None)
        ws = _WS[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
        while len(_WS) > MAX_CACHED_STREAMS:
            _WS.popitem(last=False)
    else:
        _WS.move_to_end(key)
    return ws


def release_workspaces() -> None:
    """Drop every cached workspace.  Its memory goes back to torch's caching
    allocator, which hands a block out again only to allocations on the
    stream it was allocated on, the stream whose work used it."""
    _WS.clear()


def workspace_bytes_held() -> int:
    return sum(t.numel() for t in _WS.values())
