"""Paired metadata: two adjacent 64-token query blocks share one table row.

Drop-in for reference hilberta/paired_metadata.py.  ``PairedMetadata`` is the same frozen
carrier (paired_metadata.py:8-23).  ``pair_metadata`` keeps its signature and CPU validation
(validate_metadata) but does the merge itself with the table builder, on the GPU by default or on
the host with ``device="cpu"`` (the rows become adjacency bitmaps, hb_table_bits; paired rows are
counted and emitted from them, hb_bits_counts / hb_bits_emit): for paired row r the key blocks of
query blocks 2r and 2r+1 are unioned in ascending block order and each key block gets flag bit
(half + 2*key_half) for every (query half, 64-key half) that sees it (paired_metadata.py:26-51).
Tables come back on the CPU, as in the reference, so callers keep their own ``.to(device)``
caching; ``pair_metadata_device`` keeps them where they were built.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from ._tables import _dev, emit_device, table_bits_device
from .sparse_kernel import validate_metadata


@dataclass(frozen=True)
class PairedMetadata:
    kv_indices: torch.Tensor
    kv_flags: torch.Tensor
    kv_counts: torch.Tensor
    tokens: int
    global_tokens: int
    key_block_size: int

    def to(self, device):
        return replace(
            self,
            kv_indices=self.kv_indices.to(device),
            kv_flags=self.kv_flags.to(device),
            kv_counts=self.kv_counts.to(device),
        )


def pair_tables_device(kv_indices, kv_counts, *, tokens, key_block_size):
    """Pair validated int32 tables on one device (a GPU, or the CPU for the host builder);
    returns (ids, flags, counts) on that device.

    The rows become adjacency bitmaps (hb_table_bits), paired rows are emitted in ascending key
    block order (hb_bits_counts / hb_bits_emit).  On a GPU one host synchronisation reads the
    widest paired row, which fixes the table width.
    """
    total_blocks = tokens // 64
    bits = table_bits_device(kv_indices.contiguous(), kv_counts.contiguous(), total_blocks)
    out = emit_device(bits, total_blocks, unpaired=False, paired=True, key_block_size=key_block_size)
    return out["paired_indices"], out["paired_flags"], out["paired_counts"]


def pair_metadata(kv_indices, kv_counts, *, tokens, global_tokens=768, key_block_size=64, device=None):
    """Merge two query lists; each flag bit keeps original 64x64 visibility.

    KV64 flags bits 0/1 correspond to query half 0/1.  KV128 adds bits 2/3 for query halves 0/1
    attending the block's second 64-token key half.  No key is duplicated.  All work happens once
    at plan setup, never inside attention.  The merge runs on ``device`` (default: the current
    HIP device; ``"cpu"``: the host builder); the result is returned on the CPU like the
    reference's.
    """
    validate_metadata(kv_indices, kv_counts, tokens=tokens, global_tokens=global_tokens)
    if key_block_size not in (64, 128) or tokens % 128 or global_tokens % 128:
        raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
    meta = pair_metadata_device(
        kv_indices, kv_counts, tokens=tokens, global_tokens=global_tokens,
        key_block_size=key_block_size, device=device, validated=True,
    )
    return meta.to("cpu")


def pair_metadata_device(kv_indices, kv_counts, *, tokens, global_tokens=768, key_block_size=64,
                         device=None, validated=False):
    """As pair_metadata, but the tables stay on ``device`` (on a GPU, ready for
    paired_attention)."""
    if not validated:
        validate_metadata(kv_indices, kv_counts, tokens=tokens, global_tokens=global_tokens)
        if key_block_size not in (64, 128) or tokens % 128 or global_tokens % 128:
            raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
    device = _dev(device)
    ids, flags, counts = pair_tables_device(
        kv_indices.to(device).contiguous(), kv_counts.to(device).contiguous(), tokens=tokens,
        key_block_size=key_block_size,
    )
    return PairedMetadata(ids, flags, counts, int(tokens), int(global_tokens), int(key_block_size))


def unpair_metadata(meta):
    """Reconstruct original query block lists, independently checking flags (CPU, test tooling)."""
    if any(x.device.type != "cpu" for x in (meta.kv_indices, meta.kv_flags, meta.kv_counts)):
        raise ValueError("CPU metadata required for validation")
    ratio = meta.key_block_size // 64
    rows = []
    for row, count in enumerate(meta.kv_counts.tolist()):
        ids_row = meta.kv_indices[row, :count].tolist()
        flags_row = meta.kv_flags[row, :count].tolist()
        for half in range(2):
            ids = []
            for block, flags in zip(ids_row, flags_row):
                for kh in range(ratio):
                    if flags & (1 << (half + 2 * kh)):
                        ids.append(block * ratio + kh)
            rows.append(sorted(ids))
    return rows
