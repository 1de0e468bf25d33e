"""Host-side runtime helpers of the Python wrappers (no GPU needed)."""
from __future__ import annotations

import torch

from flash_attn_volta import _runtime


def test_workspace_cache_reuses_grows_and_bounds_streams(monkeypatch):
    """Workspaces are cached per (device, stream), reused while large
    enough, replaced when a call needs more, and held for at most
    MAX_CACHED_STREAMS streams (least recently used dropped first), so a
    pool of streams cannot pin a workspace each."""
    monkeypatch.setattr(_runtime, "capturing", lambda: False)
    _runtime.release_workspaces()
    cpu = torch.device("cpu")
    a = _runtime.workspace(256, cpu, 1)
    assert _runtime.workspace(128, cpu, 1) is a              # large enough: reused
    b = _runtime.workspace(512, cpu, 1)
    assert b is not a and b.numel() == 512                   # grown
    n = _runtime.MAX_CACHED_STREAMS
    for s in range(2, n + 1):
        _runtime.workspace(64, cpu, s)
    assert len(_runtime._WS) == n
    _runtime.workspace(64, cpu, 1)                           # stream 1 most recent again
    _runtime.workspace(64, cpu, n + 1)                       # evicts stream 2, the oldest
    assert len(_runtime._WS) == n
    assert (None, 2) not in _runtime._WS and (None, 1) in _runtime._WS
    assert _runtime.workspace_bytes_held() == 512 + 64 * (n - 1)
    _runtime.release_workspaces()
    assert _runtime.workspace_bytes_held() == 0


def test_workspace_under_capture_is_fresh(monkeypatch):
    """A call made while its stream is captured into a graph gets a fresh
    tensor that the cache does not keep (the graph owns those addresses)."""
    monkeypatch.setattr(_runtime, "capturing", lambda: True)
    _runtime.release_workspaces()
    cpu = torch.device("cpu")
    a = _runtime.workspace(64, cpu, 7)
    assert _runtime.workspace(64, cpu, 7) is not a
    assert len(_runtime._WS) == 0
