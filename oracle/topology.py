"""numpy restatement of the reference's block-table topology -- TEST ORACLE ONLY.

Follows, function by function (citations into the reference checkout):
  hilbert_order          hilberta/geometry.py:6-25
  neighbor_pairs         hilberta/geometry.py:28-43
  build_plan             hilberta/plan.py:114-197
  full_attention_plan    hilberta/plan.py:200-212
  bridge_k_plan          hilberta/bridge_k.py:10-51
  pair_metadata          hilberta/paired_metadata.py:26-51
  unpair_metadata        hilberta/paired_metadata.py:54-70
  validate_metadata      hilberta/sparse_kernel.py:100-152
  dense_mask             hilberta/plan.py:70-84

Everything is integer arithmetic on numpy arrays; results are plain dicts of
numpy arrays (int64 orders, int32 tables) so they can be compared bit for bit
with the HIP builder.

Pinned by (tests/test_oracle_topology.py):
  * hilbert_order: hand case grid 2 -> [2,0,1,3]; permutation; consecutive
    entries are 4-neighbours (closed form of the Hilbert curve).
  * build_plan: known bridge budgets [24,34,32,34] / [56,57,58,55] and
    physical_original_blocks[:4] == [15,16,47,48] (reference test_plan.py:54-59);
    dense token masks equal the rolled-coordinate second algorithm in
    oracle/mask_oracle.py (reference test_plan.py:10-52 semantics).
  * bridge_k_plan: K1 == symmetrised build_plan K1 (test_bridge_k.py:9-27);
    K1..K4 == second algorithm at grid 64/128/256; 4-tile K1 bridge edges equal
    the reference's own data file website/data/demo.json (fixture copy in
    tests/golden/demo_t4k1_grid64.json); monotone in K; symmetric.
  * pair_metadata: hand vector (test_paired_metadata.py:46-55), round trip,
    popcount invariant (test_paired_metadata.py:10-44).
"""

from __future__ import annotations

import numpy as np


# --------------------------------------------------------------------------- geometry
def hilbert_order(grid_size: int = 64) -> np.ndarray:
    """Hilbert d2xy for every distance, then raster id (g-1-y)*g + x.

    Restates geometry.py:6-25 with the loop over distances vectorised.
    """
    g = int(grid_size)
    if g < 2 or g & (g - 1):
        raise ValueError("Hilbert grid side must be a power of two >= 2")
    t = np.arange(g * g, dtype=np.int64)
    x = np.zeros_like(t)
    y = np.zeros_like(t)
    s = 1
    while s < g:
        rx = (t // 2) & 1
        ry = (t ^ (t // 2)) & 1
        flip = (ry == 0) & (rx == 1)
        x = np.where(flip, s - 1 - x, x)
        y = np.where(flip, s - 1 - y, y)
        swap = ry == 0
        x, y = np.where(swap, y, x), np.where(swap, x, y)
        x = x + s * rx
        y = y + s * ry
        t = t // 4
        s *= 2
    return (g - 1 - y) * g + x


def neighbor_pairs(grid_size: int, connectivity: int = 4) -> np.ndarray:
    """Ascending undirected 4/8-neighbour pairs in (y, x, direction) order (geometry.py:28-43)."""
    if int(grid_size) != grid_size or grid_size < 1 or connectivity not in (4, 8):
        raise ValueError("positive integer grid_size and connectivity 4 or 8 required")
    g = int(grid_size)
    directions = [(0, 1), (1, 0)]
    if connectivity == 8:
        directions += [(1, 1), (1, -1)]
    yy, xx = np.meshgrid(np.arange(g), np.arange(g), indexing="ij")
    firsts, seconds, valids = [], [], []
    for dy, dx in directions:
        ny, nx = yy + dy, xx + dx
        valids.append((ny >= 0) & (ny < g) & (nx >= 0) & (nx < g))
        firsts.append(yy * g + xx)
        seconds.append(ny * g + nx)
    # stack along a trailing direction axis so flattening walks y, x, direction
    first = np.stack(firsts, -1).reshape(-1)
    second = np.stack(seconds, -1).reshape(-1)
    valid = np.stack(valids, -1).reshape(-1)
    return np.stack((first[valid], second[valid]), 1).astype(np.int64)


# --------------------------------------------------------------------------- plan
def _check_positive_ints(**values):
    for name, value in values.items():
        if isinstance(value, bool) or int(value) != value or value <= 0:
            raise ValueError(f"{name} must be a positive integer")


def _pair_scores(inverse, labels, pairs, block_size, nb):
    """Symmetric count of cross-tile 4-neighbour pairs per (query block, key block).

    plan.py:159-165 and bridge_k.py:22-28: for every missing pair (a, c) the
    counter gets (blk(a), blk(c)) += 1 and (blk(c), blk(a)) += 1.
    """
    missing = pairs[labels[pairs[:, 0]] != labels[pairs[:, 1]]]
    ba = inverse[missing[:, 0]] // block_size
    bc = inverse[missing[:, 1]] // block_size
    scores = np.zeros((nb, nb), dtype=np.int64)
    np.add.at(scores, (ba, bc), 1)
    np.add.at(scores, (bc, ba), 1)
    return scores


def _top_keys(scores, q, k, offset_blocks, nb):
    """Top-k keys of row q by (-score, (key - offset_blocks) mod nb) (bridge_k.py:36-40)."""
    keys = np.nonzero(scores[q])[0]
    if len(keys) == 0:
        return []
    rolled = (keys - offset_blocks) % nb
    order = np.lexsort((rolled, -scores[q, keys]))
    return [int(x) for x in keys[order[:k]]]


def build_plan(tile_count=4, grid_size=64, text_tokens=512, shared=True, bridge=True, block_size=64):
    """Restates plan.py:114-197; returns a dict mirroring AttentionPlan fields."""
    _check_positive_ints(
        tile_count=tile_count, grid_size=grid_size, text_tokens=text_tokens, block_size=block_size
    )
    tile_count, grid_size, text_tokens, block_size = map(
        int, (tile_count, grid_size, text_tokens, block_size)
    )
    n = grid_size**2
    if grid_size < 8 or grid_size & (grid_size - 1):
        raise ValueError("grid_size must be a power of two >= 8")
    if n % tile_count or (n // tile_count) % (4 * block_size) or text_tokens % block_size:
        raise ValueError("Tile quarter offsets and text prefix must be block aligned")
    h = hilbert_order(grid_size)
    mid = h[n // 4 : 3 * n // 4]
    original = np.concatenate((mid, n - 1 - mid))  # plan.py:134
    inverse = np.argsort(original, kind="stable")  # plan.py:135
    blocks = original.reshape(-1, block_size)
    nb = len(blocks)
    shared_ids = np.zeros(n, dtype=bool)
    if shared:  # plan.py:139-141
        start, end = 3 * grid_size // 8, 5 * grid_size // 8
        shared_ids.reshape(grid_size, grid_size)[start:end, start:end] = True
    share_counts = shared_ids[blocks].sum(1)
    if ((share_counts != 0) & (share_counts != block_size)).any():
        raise ValueError("Shared square must be a union of complete original blocks")
    share_blocks = np.nonzero(share_counts == block_size)[0]
    ordinary = np.nonzero(share_counts == 0)[0]
    packed_blocks = np.concatenate((share_blocks, ordinary))  # plan.py:146
    order = blocks[packed_blocks].reshape(-1)
    original_to_physical = np.argsort(packed_blocks, kind="stable") + text_tokens // block_size
    global_blocks = text_tokens // block_size + len(share_blocks)
    pairs = neighbor_pairs(grid_size, 4)
    width = n // tile_count
    phases = []
    for offset in (0, width // 4, width // 2, 3 * width // 4):  # plan.py:154
        labels = ((inverse - offset) % n) // width
        block_labels = labels[blocks[:, 0]]
        if not np.array_equal(labels[blocks], np.broadcast_to(block_labels[:, None], blocks.shape)):
            raise AssertionError("A physical block crosses a tile boundary")
        chosen = np.full(nb, -1, dtype=np.int64)
        if bridge:  # plan.py:159-172: directed top-1, no symmetrisation
            scores = _pair_scores(inverse, labels, pairs, block_size, nb)
            for q in range(nb):
                top = _top_keys(scores, q, 1, offset // block_size, nb)
                if top:
                    chosen[q] = top[0]
        rows = []
        for q in ordinary.tolist():  # plan.py:173-183
            same_tile = ordinary[block_labels[ordinary] == block_labels[q]]
            keys = set(range(global_blocks)) | set(original_to_physical[same_tile].tolist())
            if chosen[q] >= 0:
                keys.add(int(original_to_physical[chosen[q]]))
            rows.append(sorted(keys))
        counts = np.array([len(r) for r in rows], dtype=np.int32)
        indices = np.zeros((len(rows), int(counts.max())), dtype=np.int32)
        for q, row in enumerate(rows):
            indices[q, : len(row)] = row
        phases.append(
            dict(offset=offset, kv_indices=indices, kv_counts=counts, bridge_original_blocks=chosen)
        )
    return dict(
        grid_size=grid_size,
        tile_count=tile_count,
        text_tokens=text_tokens,
        shared_tokens=len(share_blocks) * block_size,
        block_size=block_size,
        image_order=order.astype(np.int64),
        inverse_image_order=np.argsort(order, kind="stable").astype(np.int64),
        original_order=original.astype(np.int64),
        physical_original_blocks=packed_blocks.astype(np.int64),
        phases=phases,
        bridge=bool(bridge),
        full=False,
        image_tokens=n,
        global_tokens=text_tokens + len(share_blocks) * block_size,
        total_tokens=text_tokens + n,
    )


def full_attention_plan(plan):
    """All-connection tables over the same layout (plan.py:200-212)."""
    nb = plan["total_tokens"] // plan["block_size"]
    nq = (plan["total_tokens"] - plan["global_tokens"]) // plan["block_size"]
    ids = np.tile(np.arange(nb, dtype=np.int32), (nq, 1))
    counts = np.full(nq, nb, dtype=np.int32)
    out = dict(plan)
    out["phases"] = [dict(p, kv_indices=ids.copy(), kv_counts=counts.copy()) for p in plan["phases"]]
    out["full"] = True
    return out


def bridge_k_plan(tiles=4, k=1, shared=False, *, grid_size=64):
    """Restates bridge_k.py:10-51: top-K reciprocal block bridges on a bridge-free base plan."""
    if isinstance(k, bool) or k not in (1, 2, 3, 4):
        raise ValueError("This bounded comparison supports integer K=1..4")
    plan = build_plan(tiles, grid_size=grid_size, shared=shared, bridge=False)
    n = plan["image_tokens"]
    b = plan["block_size"]
    nb = n // b
    g = plan["global_tokens"] // b
    inverse = np.argsort(plan["original_order"], kind="stable")
    physical = np.argsort(plan["physical_original_blocks"], kind="stable") + plan["text_tokens"] // b
    pairs = neighbor_pairs(plan["grid_size"], 4)
    total_blocks = plan["total_tokens"] // b
    phases = []
    for p in plan["phases"]:
        labels = ((inverse - p["offset"]) % n) // (n // tiles)
        scores = _pair_scores(inverse, labels, pairs, b, nb)
        chosen = np.full((nb, k), -1, dtype=np.int64)
        adj = np.zeros((total_blocks, total_blocks), dtype=bool)  # bridge_k.py:31-35
        adj[:g, :] = True
        for row, count in enumerate(p["kv_counts"].tolist()):
            adj[g + row, p["kv_indices"][row, :count]] = True
        for q in range(nb):  # bridge_k.py:36-43
            for j, key in enumerate(_top_keys(scores, q, k, p["offset"] // b, nb)):
                chosen[q, j] = key
                adj[physical[q], physical[key]] = True
        adj = adj | adj.T  # bridge_k.py:44
        rows = [np.nonzero(adj[q])[0].astype(np.int32) for q in range(g, total_blocks)]
        sizes = np.array([len(r) for r in rows], dtype=np.int32)
        ids = np.zeros((len(rows), int(sizes.max())), dtype=np.int32)
        for q, row in enumerate(rows):
            ids[q, : len(row)] = row
        phases.append(
            dict(offset=p["offset"], kv_indices=ids, kv_counts=sizes, bridge_original_blocks=chosen)
        )
    out = dict(plan)
    out["phases"] = phases
    out["bridge"] = True
    return out


def block_adjacency(plan, phase):
    """Physical block adjacency [T, T] bool of one phase: global rows all True, ordinary rows from tables."""
    b = plan["block_size"]
    total_blocks = plan["total_tokens"] // b
    g = plan["global_tokens"] // b
    p = plan["phases"][phase % 4]
    adj = np.zeros((total_blocks, total_blocks), dtype=bool)
    adj[:g] = True
    for row, count in enumerate(p["kv_counts"].tolist()):
        adj[g + row, p["kv_indices"][row, :count]] = True
    return adj


def dense_mask(plan, phase):
    """Token-level physical mask [N, N] (plan.py:70-84)."""
    b = plan["block_size"]
    return block_adjacency(plan, phase).repeat(b, 0).repeat(b, 1)


# --------------------------------------------------------------------------- metadata
def validate_metadata(kv_indices, kv_counts, *, tokens, global_tokens=768, block_size=64,
                      require_global_prefix=True):
    """Restates the value checks of sparse_kernel.py:100-152 on numpy tables."""
    if block_size != 64:
        raise ValueError("This kernel currently requires 64-token physical blocks")
    if not (0 <= global_tokens < tokens) or tokens % block_size or global_tokens % block_size:
        raise ValueError("tokens/global prefix must be block-aligned with at least one ordinary block")
    kv_indices = np.asarray(kv_indices)
    kv_counts = np.asarray(kv_counts)
    if kv_indices.dtype != np.int32 or kv_counts.dtype != np.int32:
        raise TypeError("Block metadata must use int32")
    rows = (tokens - global_tokens) // block_size
    if kv_indices.ndim != 2 or kv_indices.shape[0] != rows or kv_indices.shape[1] < 1:
        raise ValueError("kv_indices must be [ordinary_query_blocks, max_KV_blocks]")
    if kv_counts.shape != (rows,):
        raise ValueError("kv_counts must have one entry per ordinary query block")
    nblocks, global_blocks = tokens // block_size, global_tokens // block_size
    for row, count in enumerate(kv_counts.tolist()):
        if not 1 <= count <= kv_indices.shape[1]:
            raise ValueError(f"Invalid K/V count in ordinary query block {row}")
        ids = kv_indices[row, :count]
        if ids.min() < 0 or ids.max() >= nblocks or len(set(ids.tolist())) != count:
            raise ValueError(f"Out-of-range or duplicate K/V blocks in row {row}")
        if require_global_prefix and not set(range(global_blocks)).issubset(ids.tolist()):
            raise ValueError(f"Row {row} misses global-prefix keys")
    ordinary_entries = int(kv_counts.sum()) * block_size * block_size
    return dict(
        tokens=tokens,
        global_tokens=global_tokens,
        block_size=block_size,
        ordinary_query_blocks=rows,
        min_kv_blocks=int(kv_counts.min()),
        max_kv_blocks=int(kv_counts.max()),
        global_directed_entries=global_tokens * tokens,
        ordinary_directed_entries=ordinary_entries,
        total_directed_entries=global_tokens * tokens + ordinary_entries,
    )


def pair_metadata(kv_indices, kv_counts, *, tokens, global_tokens=768, key_block_size=64):
    """Merge query blocks 2r and 2r+1; flag bit (half + 2*key_half) (paired_metadata.py:26-51)."""
    validate_metadata(kv_indices, kv_counts, tokens=tokens, global_tokens=global_tokens)
    if key_block_size not in (64, 128) or tokens % 128 or global_tokens % 128:
        raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
    kv_indices = np.asarray(kv_indices)
    kv_counts = np.asarray(kv_counts)
    ratio = key_block_size // 64
    rows = []
    for q in range(0, len(kv_counts), 2):
        union = {}
        for half in range(2):
            for block in kv_indices[q + half, : int(kv_counts[q + half])].tolist():
                block_id, key_half = divmod(block, ratio)
                union[block_id] = union.get(block_id, 0) | (1 << (half + 2 * key_half))
        rows.append(sorted(union.items()))
    counts = np.array([len(x) for x in rows], dtype=np.int32)
    ids = np.zeros((len(rows), int(counts.max())), dtype=np.int32)
    flags = np.zeros_like(ids)
    for q, row in enumerate(rows):
        for j, (block, flag) in enumerate(row):
            ids[q, j], flags[q, j] = block, flag
    return dict(kv_indices=ids, kv_flags=flags, kv_counts=counts, tokens=tokens,
                global_tokens=global_tokens, key_block_size=key_block_size)


def unpair_metadata(meta):
    """Original per-query-block lists recovered from paired flags (paired_metadata.py:54-70)."""
    ratio = meta["key_block_size"] // 64
    rows = []
    for row, count in enumerate(np.asarray(meta["kv_counts"]).tolist()):
        ids_row = meta["kv_indices"][row, :count].tolist()
        flags_row = meta["kv_flags"][row, :count].tolist()
        for half in range(2):
            ids = []
            for block, flags in zip(ids_row, flags_row):
                for kh in range(ratio):
                    if flags & (1 << (half + 2 * kh)):
                        ids.append(block * ratio + kh)
            rows.append(sorted(ids))
    return rows


def live_blocks(plan, phase):
    """Live 64x64 blocks of one phase = G*T + sum(counts) (plan.py:103-106 directed_entries / 64^2)."""
    b = plan["block_size"]
    g = plan["global_tokens"] // b
    total = plan["total_tokens"] // b
    return g * total + int(plan["phases"][phase % 4]["kv_counts"].sum())
