"""Static block plans: composite Hilbert order, sliding tiles, bridges (drop-in for reference plan.py).

Physical stream is [text, shared image blocks, remaining image blocks].  Tile membership and
bridge tie breaking use the ORIGINAL phase ordering.  ``PhasePlan`` / ``AttentionPlan`` are the
reference's carriers (plan.py:17-111).  ``build_plan`` keeps its signature, validation and
results (plan.py:114-197) but the tables are built on the GPU by csrc/tables.hip (or on the host
by csrc/tables_host.hip with ``device="cpu"``) and returned on the CPU; ``full_attention_plan``
(plan.py:200-212) is host bookkeeping.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, replace

import torch

from ._tables import emit_device_many, layout_device, phase_bits_device


@dataclass(frozen=True)
class PhasePlan:
    offset: int
    kv_indices: torch.Tensor
    kv_counts: torch.Tensor
    bridge_original_blocks: torch.Tensor

    def to(self, device):
        return replace(
            self,
            kv_indices=self.kv_indices.to(device),
            kv_counts=self.kv_counts.to(device),
            bridge_original_blocks=self.bridge_original_blocks.to(device),
        )


@dataclass(frozen=True)
class AttentionPlan:
    grid_size: int
    tile_count: int
    text_tokens: int
    shared_tokens: int
    block_size: int
    image_order: torch.Tensor
    inverse_image_order: torch.Tensor
    original_order: torch.Tensor
    physical_original_blocks: torch.Tensor
    phases: tuple
    bridge: bool
    full: bool = False

    @property
    def image_tokens(self):
        return self.grid_size**2

    @property
    def global_tokens(self):
        return self.text_tokens + self.shared_tokens

    @property
    def total_tokens(self):
        return self.text_tokens + self.image_tokens

    def to(self, device):
        return replace(
            self,
            image_order=self.image_order.to(device),
            inverse_image_order=self.inverse_image_order.to(device),
            original_order=self.original_order.to(device),
            physical_original_blocks=self.physical_original_blocks.to(device),
            phases=tuple(p.to(device) for p in self.phases),
        )

    def dense_mask(self, phase, device=None):
        """Explicit physical-identity mask for correctness only (plan.py:70-84)."""
        p = self.phases[phase % 4]
        device = p.kv_indices.device if device is None else device
        total = self.total_tokens // self.block_size
        glob = self.global_tokens // self.block_size
        blocks = torch.zeros(total, total, dtype=torch.bool)
        blocks[:glob] = True
        ids, counts = p.kv_indices.cpu().long(), p.kv_counts.cpu()
        active = torch.arange(ids.shape[1])[None, :] < counts[:, None]
        rows = torch.arange(len(counts))[:, None].expand_as(ids)
        blocks[glob + rows[active], ids[active]] = True
        return (
            blocks.repeat_interleave(self.block_size, 0)
            .repeat_interleave(self.block_size, 1)
            .to(device)
        )

    def manifest(self):
        """JSON-ready summary in the reference's manifest format (plan.py:86-111): the geometry
        fields, a SHA-256 of the image order's int64 bytes, the physical block packing and, per
        phase, its offset, the range of row lengths, the directed (query, key) token entries
        the tables admit and the chosen bridge blocks."""
        bs = self.block_size
        # every global query block sees every key block; ordinary rows see what they list
        global_block_entries = (self.global_tokens // bs) * (self.total_tokens // bs)

        def phase_summary(p):
            counts = p.kv_counts.cpu()
            listed = int(counts.sum())
            return {
                "offset": p.offset,
                "kv_count_min": int(counts.min()),
                "kv_count_max": int(counts.max()),
                "directed_entries": (global_block_entries + listed) * bs * bs,
                "bridge_original_blocks": p.bridge_original_blocks.cpu().tolist(),
            }

        fields = ("grid_size", "tile_count", "text_tokens", "shared_tokens", "block_size", "bridge",
                  "full")
        summary = {name: getattr(self, name) for name in fields}
        summary["image_order_sha256"] = hashlib.sha256(
            self.image_order.cpu().numpy().tobytes()).hexdigest()
        summary["physical_original_blocks"] = self.physical_original_blocks.cpu().tolist()
        summary["phases"] = [phase_summary(p) for p in self.phases]
        return summary


def _check_geometry(tile_count, grid_size, text_tokens, block_size):
    for name, value in [
        ("tile_count", tile_count),
        ("grid_size", grid_size),
        ("text_tokens", text_tokens),
        ("block_size", block_size),
    ]:
        if isinstance(value, bool) or int(value) != value or value <= 0:
            raise ValueError(f"{name} must be a positive integer")
    tile_count, grid_size, text_tokens, block_size = map(
        int, (tile_count, grid_size, text_tokens, block_size)
    )
    n = grid_size**2
    if grid_size < 8 or grid_size & (grid_size - 1):
        raise ValueError("grid_size must be a power of two >= 8")
    if n % tile_count or (n // tile_count) % (4 * block_size) or text_tokens % block_size:
        raise ValueError("Tile quarter offsets and text prefix must be block aligned")
    return tile_count, grid_size, text_tokens, block_size


def _device_plan(tile_count, grid_size, text_tokens, shared, bridge_mode, k, block_size, device):
    layout = layout_device(grid_size, block_size, text_tokens, shared, device)
    scratch = None
    if bridge_mode:
        scratch = torch.empty(layout.image_blocks**2, dtype=torch.int32,
                              device=layout.original_order.device)
    width = grid_size**2 // tile_count
    built = [phase_bits_device(layout, tile_count, phase, bridge_mode, k, scratch)
             for phase in range(4)]
    tables = emit_device_many([b for b, _ in built], layout.total_blocks, unpaired=True)
    return layout, [(phase * (width // 4), bits, t, chosen)
                    for phase, ((bits, chosen), t) in enumerate(zip(built, tables))]


def build_plan(tile_count=4, grid_size=64, text_tokens=512, shared=True, bridge=True, block_size=64,
               *, device=None):
    """Build the static plan on ``device`` (default: the current HIP device; ``"cpu"``: the host
    builder); the returned AttentionPlan holds CPU tensors."""
    tile_count, grid_size, text_tokens, block_size = _check_geometry(
        tile_count, grid_size, text_tokens, block_size
    )
    layout, phases = _device_plan(tile_count, grid_size, text_tokens, shared, 1 if bridge else 0, 1,
                                  block_size, device)
    return _to_attention_plan(layout, phases, tile_count, bool(bridge), directed=True)


def _to_attention_plan(layout, phases, tile_count, bridge, directed):
    phase_plans = []
    for offset, _bits, tables, chosen in phases:
        chosen = chosen.cpu()
        if directed:
            chosen = chosen[:, 0].clone()
        phase_plans.append(
            PhasePlan(offset, tables["kv_indices"].cpu(), tables["kv_counts"].cpu(), chosen)
        )
    return AttentionPlan(
        layout.grid_size,
        tile_count,
        layout.text_tokens,
        layout.shared_blocks * layout.block_size,
        layout.block_size,
        layout.image_order.cpu(),
        layout.inverse_image_order.cpu(),
        layout.original_order.cpu(),
        layout.physical_original_blocks.cpu(),
        tuple(phase_plans),
        bridge,
    )


def full_attention_plan(plan):
    """The same persistent layout with every ordinary query block listing every key block
    (plan.py:200-212): the dense gate, equal to unmasked attention up to the permutation."""
    key_blocks = plan.total_tokens // plan.block_size
    rows = (plan.total_tokens - plan.global_tokens) // plan.block_size

    def every_block(p):
        ids = torch.arange(key_blocks, dtype=torch.int32).expand(rows, key_blocks).contiguous()
        return replace(p, kv_indices=ids, kv_counts=torch.full((rows,), key_blocks, dtype=torch.int32))

    return replace(plan, phases=tuple(every_block(p) for p in plan.phases), full=True)
