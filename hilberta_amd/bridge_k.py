"""Top-K reciprocal block bridges (drop-in for reference hilberta/bridge_k.py).

``bridge_k_plan`` keeps the reference's signature and results (bridge_k.py:10-51): per phase,
every query block takes its K best key blocks by (-score, (key - offset/64) mod nb), where the
score counts cross-tile 4-neighbour token pairs between the two blocks, and the block adjacency is
closed under transposition.  The tables are built on the GPU (csrc/tables.hip, bridge mode 2),
or on the host with ``device="cpu"`` (csrc/tables_host.hip), and returned on the CPU.
``paired_plan_device`` is the all-device fast path: it emits the four phases' paired tables
straight from the adjacency bitmaps, ready for ``paired_attention``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .paired_metadata import PairedMetadata
from .plan import _check_geometry, _device_plan, _to_attention_plan
from ._tables import DeviceLayout, paired_plan_tables_device


def _check_k(k):
    if isinstance(k, bool) or k not in (1, 2, 3, 4):
        raise ValueError("This bounded comparison supports integer K=1..4")


def bridge_k_plan(tiles=4, k=1, shared=False, *, grid_size=64, device=None):
    _check_k(k)
    tiles, grid_size, text_tokens, block_size = _check_geometry(tiles, grid_size, 512, 64)
    layout, phases = _device_plan(tiles, grid_size, text_tokens, shared, 2, k, block_size, device)
    return _to_attention_plan(layout, phases, tiles, True, directed=False)


@dataclass
class DevicePlan:
    """Device-resident layout plus the four phases' paired tables."""

    layout: DeviceLayout
    tile_count: int
    k: int
    phases: list  # PairedMetadata per phase, tables on the device

    @property
    def total_tokens(self):
        return self.layout.text_tokens + self.layout.image_tokens

    @property
    def global_tokens(self):
        return self.layout.global_blocks * self.layout.block_size


def paired_plan_device(tiles=4, k=1, shared=False, *, grid_size=64, text_tokens=512,
                       key_block_size=64, device=None):
    """bridge_k_plan + pair_metadata for all four phases without leaving the GPU: six launches and
    one host read (_tables.paired_plan_tables_device).  ``device="cpu"`` builds the same tables
    on the host."""
    _check_k(k)
    tiles, grid_size, text_tokens, block_size = _check_geometry(tiles, grid_size, text_tokens, 64)
    if key_block_size not in (64, 128) or (text_tokens + grid_size**2) % 128:
        raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
    layout, tables = paired_plan_tables_device(grid_size, tiles, k, text_tokens, shared,
                                               key_block_size, device)
    N = text_tokens + grid_size**2
    G = layout.global_blocks * block_size
    metas = [PairedMetadata(ids, flags, counts, N, G, key_block_size) for ids, flags, counts in tables]
    return DevicePlan(layout, tiles, k, metas)
