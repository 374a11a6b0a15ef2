"""CPU checks of the drop-in surface's host functions: neighbor_pairs, explicit_mask,
AttentionPlan.manifest and full_attention_plan.

References: the oracle (oracle/topology.py, oracle/attention.py), a brute-force enumeration of
grid neighbours, and the dense mask itself (its number of true entries is the number of directed
(query, key) entries a manifest reports, reference tests/test_paired_metadata.py:36-44).
"""

import json

import numpy as np
import pytest
import torch

from hilberta_amd.geometry import neighbor_pairs
from hilberta_amd.plan import AttentionPlan, PhasePlan, full_attention_plan
from hilberta_amd.sparse_kernel import explicit_mask
from oracle import attention as A
from oracle import topology as T


def _brute_neighbours(g, connectivity):
    """Each cell in raster order, then its right, down (and down-right, down-left) neighbour."""
    steps = [(0, 1), (1, 0)] + ([(1, 1), (1, -1)] if connectivity == 8 else [])
    out = []
    for y in range(g):
        for x in range(g):
            for dy, dx in steps:
                if 0 <= y + dy < g and 0 <= x + dx < g:
                    out.append((y * g + x, (y + dy) * g + x + dx))
    return np.array(out, dtype=np.int64).reshape(-1, 2)


@pytest.mark.parametrize("connectivity", [4, 8])
def test_neighbor_pairs(connectivity):
    for g in (1, 2, 3, 5, 8, 16):
        got = neighbor_pairs(g, connectivity)
        assert got.dtype == torch.int64
        assert np.array_equal(got.numpy(), _brute_neighbours(g, connectivity)), g
    for g in (64, 128, 256):
        got = neighbor_pairs(g, connectivity).numpy()
        assert np.array_equal(got, T.neighbor_pairs(g, connectivity)), g
    with pytest.raises(ValueError):
        neighbor_pairs(0)
    with pytest.raises(ValueError):
        neighbor_pairs(8, 6)


def _plan(name_args, *, full=False):
    """AttentionPlan assembled from the oracle's plan (CPU tensors, no GPU)."""
    tiles, k, grid = name_args
    o = T.bridge_k_plan(tiles, k, False, grid_size=grid)
    if full:
        o = T.full_attention_plan(o)
    t = torch.from_numpy
    phases = tuple(PhasePlan(p["offset"], t(p["kv_indices"]), t(p["kv_counts"]),
                             t(p["bridge_original_blocks"])) for p in o["phases"])
    plan = AttentionPlan(o["grid_size"], o["tile_count"], o["text_tokens"], o["shared_tokens"],
                         o["block_size"], t(o["image_order"]), t(o["inverse_image_order"]),
                         t(o["original_order"]), t(o["physical_original_blocks"]), phases, o["bridge"],
                         o["full"])
    return plan, o


@pytest.mark.parametrize("args", [(16, 3, 64), (4, 1, 64)])
def test_explicit_mask_equals_oracle(args):
    plan, o = _plan(args)
    N, G = o["total_tokens"], o["global_tokens"]
    for p in plan.phases:
        got = explicit_mask(p.kv_indices, p.kv_counts, tokens=N, global_tokens=G)
        ref = A.explicit_mask(p.kv_indices.numpy(), p.kv_counts.numpy(), tokens=N, global_tokens=G)
        assert got.dtype == torch.bool and got.shape == (N, N)
        assert torch.equal(got, ref)
    bad = plan.phases[0].kv_indices.clone()
    bad[0, 0] = bad[0, 1]
    with pytest.raises(ValueError, match="duplicate"):
        explicit_mask(bad, plan.phases[0].kv_counts, tokens=N, global_tokens=G)


@pytest.mark.parametrize("args", [(16, 3, 64), (4, 1, 64)])
def test_manifest_counts_the_mask(args):
    plan, o = _plan(args)
    N, G = o["total_tokens"], o["global_tokens"]
    m = plan.manifest()
    assert list(m) == ["grid_size", "tile_count", "text_tokens", "shared_tokens", "block_size",
                       "bridge", "full", "image_order_sha256", "physical_original_blocks", "phases"]
    assert (m["grid_size"], m["tile_count"], m["block_size"], m["bridge"], m["full"]) == (
        args[2], args[0], 64, True, False)
    assert m["physical_original_blocks"] == o["physical_original_blocks"].tolist()
    import hashlib

    assert m["image_order_sha256"] == hashlib.sha256(
        np.asarray(o["image_order"], dtype=np.int64).tobytes()).hexdigest()
    json.dumps(m)  # JSON-ready
    for p, pm, op in zip(plan.phases, m["phases"], o["phases"]):
        mask = A.explicit_mask(op["kv_indices"], op["kv_counts"], tokens=N, global_tokens=G)
        assert pm["directed_entries"] == int(mask.sum())
        assert pm["offset"] == op["offset"]
        assert (pm["kv_count_min"], pm["kv_count_max"]) == (op["kv_counts"].min(), op["kv_counts"].max())
        assert pm["bridge_original_blocks"] == op["bridge_original_blocks"].tolist()


def test_full_attention_plan():
    plan, o = _plan((16, 3, 64))
    full = full_attention_plan(plan)
    ref = T.full_attention_plan(o)
    N = plan.total_tokens
    assert full.full and not plan.full
    assert torch.equal(full.image_order, plan.image_order)
    for p, rp in zip(full.phases, ref["phases"]):
        assert p.kv_indices.dtype == torch.int32 and p.kv_indices.is_contiguous()
        assert np.array_equal(p.kv_indices.numpy(), rp["kv_indices"])
        assert np.array_equal(p.kv_counts.numpy(), rp["kv_counts"])
    assert all(pm["directed_entries"] == N * N for pm in full.manifest()["phases"])
    # the phases hold tables of their own
    assert full.phases[0].kv_indices.data_ptr() != full.phases[1].kv_indices.data_ptr()
