"""Shared test helpers: oracle-built tables as test inputs and the parity comparison."""

from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import attention as A
from oracle import topology as T

# Tolerances of the attention path against the fp32 dense masked reference.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3
LSE_ABS = 1e-3

CONFIGS = {
    # name: (grid, tiles, K)
    "1024_t4k1": (64, 4, 1),
    "1024_t16k3": (64, 16, 3),
    "2048_t4k1": (128, 4, 1),
    "2048_t16k3": (128, 16, 3),
    "4096_t16k3": (256, 16, 3),
}


def say(*args):
    """Print and flush, so a GPU step that dies still names its case."""
    print(*args, flush=True)
    sys.stdout.flush()


_PLAN_CACHE: dict = {}


def oracle_plan(name):
    if name not in _PLAN_CACHE:
        grid, tiles, k = CONFIGS[name]
        _PLAN_CACHE[name] = T.bridge_k_plan(tiles, k, False, grid_size=grid)
    return _PLAN_CACHE[name]


def oracle_paired(plan, phase, key_block_size=64):
    p = plan["phases"][phase]
    return T.pair_metadata(p["kv_indices"], p["kv_counts"], tokens=plan["total_tokens"],
                           global_tokens=plan["global_tokens"], key_block_size=key_block_size)


def device_paired(meta_np, device):
    """PairedMetadata on the device built from numpy oracle tables (a test input)."""
    from hilberta_amd.paired_metadata import PairedMetadata

    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)  # noqa: E731
    return PairedMetadata(t(meta_np["kv_indices"]), t(meta_np["kv_flags"]), t(meta_np["kv_counts"]),
                          int(meta_np["tokens"]), int(meta_np["global_tokens"]),
                          int(meta_np["key_block_size"]))


def compare(out, lse, ref_out, ref_lse, what, rows=None):
    """Assert the tolerance bar; returns (max_abs, mean_abs, lse_abs)."""
    o = out.float()
    r = ref_out.to(o.device)
    if rows is not None:
        o, r = o[:, :, rows], r[:, :, rows]
    diff = (o - r).abs()
    assert torch.isfinite(o).all(), f"{what}: non-finite output"
    max_abs, mean_abs = diff.max().item(), diff.mean().item()
    lse_abs = 0.0
    if lse is not None:
        l, rl = lse, ref_lse.to(lse.device)
        if rows is not None:
            l, rl = l[:, :, rows], rl[:, :, rows]
        lse_abs = (l - rl).abs().max().item()
    say(f"{what}: max_abs={max_abs:.3e} mean_abs={mean_abs:.3e} lse_abs={lse_abs:.3e}")
    assert max_abs <= MAX_ABS, f"{what}: max abs {max_abs}"
    assert mean_abs <= MEAN_ABS, f"{what}: mean abs {mean_abs}"
    assert lse_abs <= LSE_ABS, f"{what}: lse abs {lse_abs}"
    return max_abs, mean_abs, lse_abs


def reference(q, k, v, plan, phase, heads=None, device="cpu"):
    """fp32 oracle output/LSE for a plan phase (block formulation; no N x N mask)."""
    p = plan["phases"][phase]
    return A.block_sparse_attention(q.to(device), k.to(device), v.to(device), p["kv_indices"],
                                    p["kv_counts"], global_tokens=plan["global_tokens"], heads=heads)


def eq_exact(a, b, what):
    """Bit-exact comparison of a table (tensor on any device, or array) with an oracle array."""
    a = a.cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    assert a.dtype == b.dtype or (a.dtype.kind == b.dtype.kind == "i"), f"{what}: dtype {a.dtype} {b.dtype}"
    assert np.array_equal(a, b), f"{what}: values differ at {np.argwhere(a != b)[:5].tolist()}"


def plan_eq(dev, ref, what, directed):
    """An AttentionPlan against the oracle's plan dict: geometry, orders, every phase's tables."""
    assert dev.grid_size == ref["grid_size"] and dev.tile_count == ref["tile_count"]
    assert dev.shared_tokens == ref["shared_tokens"] and dev.global_tokens == ref["global_tokens"]
    for f in ("image_order", "inverse_image_order", "original_order", "physical_original_blocks"):
        eq_exact(getattr(dev, f), ref[f], f"{what} {f}")
        assert getattr(dev, f).dtype == torch.int64
    for i, (p, r) in enumerate(zip(dev.phases, ref["phases"])):
        assert p.offset == r["offset"]
        assert p.kv_indices.dtype == torch.int32 and p.kv_counts.dtype == torch.int32
        eq_exact(p.kv_indices, r["kv_indices"], f"{what} phase {i} kv_indices")
        eq_exact(p.kv_counts, r["kv_counts"], f"{what} phase {i} kv_counts")
        eq_exact(p.bridge_original_blocks, r["bridge_original_blocks"], f"{what} phase {i} bridges")
