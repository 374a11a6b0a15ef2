"""Per-(device, stream) workspaces for the attention kernels.

A workspace holds the persistent kernel's work-queue counters (zero-filled once at allocation;
every launch leaves them at zero) and the partial results of split global query tiles.  Keying
by stream keeps launches that may overlap in time from sharing one.
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
    stream = torch.cuda.current_stream(device)
    key = (str(device), stream.cuda_stream)
    ws = _CACHE.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=device)
        _CACHE[key] = ws
    return ws


def clear() -> None:
    _CACHE.clear()
