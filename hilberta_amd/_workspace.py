"""Per-(device, stream) workspaces for the attention kernels.

A workspace holds the persistent kernel's work-queue counters (zero-filled once at allocation;
every launch leaves them at zero) and the partial results of split global query tiles.  Keying
by stream keeps launches that may overlap in time from sharing one.

A launch captured into a HIP graph gets a workspace of its own, made during the capture with a
fill kernel (so every replay zero-fills it before the attention kernel runs) and released when the
launch returns: it comes from the capture's private memory pool, which the graph keeps alive, and
later allocations of the same capture may reuse it only in stream order, after this launch's
kernels.  Captured launches therefore hold no memory beyond their graph's lifetime.
"""

from __future__ import annotations

import torch

from . import _lib

_CACHE: dict = {}


def attention_workspace(device, batch, heads, tokens, head_dim, global_tokens, width,
                        key_block_size, *, paired, all_queries):
    need = _lib.load().hb_attention_workspace_bytes(
        batch, heads, tokens, head_dim, global_tokens, width, key_block_size, int(paired),
        int(all_queries))
    if need < 0:
        _lib.check(1, "hb_attention_workspace_bytes")
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)
    key = (str(device), stream.cuda_stream)
    ws = _CACHE.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=device)
        _CACHE[key] = ws
    return ws


def clear() -> None:
    """Drop the cached eager workspaces."""
    _CACHE.clear()
