"""Per-(device, stream, graph capture) workspaces for the attention kernels.

A workspace holds the persistent kernel's work-queue counters (zero-filled once at allocation;
every launch leaves them at zero) and the partial results of split global query tiles.  Keying
by stream keeps launches that may overlap in time from sharing one; launches captured into a HIP
graph get a workspace per capture (graphs captured one after another on the same stream may be
replayed concurrently later), made during the capture, so every replay zero-fills it first, and
kept for the life of the process since the graph may be replayed at any time.
"""

from __future__ import annotations

import torch

from . import _lib

_CACHE: dict = {}
# every workspace a captured launch uses: graphs keep pointing at them after the cache moves on
_CAPTURED: list = []


def attention_workspace(device, batch, heads, tokens, head_dim, global_tokens, width,
                        key_block_size, *, paired, all_queries):
    need = _lib.load().hb_attention_workspace_bytes(
        batch, heads, tokens, head_dim, global_tokens, width, key_block_size, int(paired),
        int(all_queries))
    if need < 0:
        _lib.check(1, "hb_attention_workspace_bytes")
    stream = torch.cuda.current_stream(device)
    capture = _lib.capture_id(stream.cuda_stream) if torch.cuda.is_current_stream_capturing() else 0
    key = (str(device), stream.cuda_stream, capture)
    ws = _CACHE.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=device)
        _CACHE[key] = ws
        if capture:
            _CAPTURED.append(ws)
    return ws


def clear() -> None:
    """Drop the cached eager workspaces (those of captured graphs stay alive)."""
    _CACHE.clear()
