"""Second, ordering-independent topology algorithm -- TEST ORACLE ONLY.

Restates the semantics of the reference's tests/topology_oracle.py
(_setup :33-52, base_masks :55-58, augmentation_masks "block_bridge" :308-329)
in numpy. It works in the phase-ROLLED sequence (order.roll(-offset)), counts
missing 4-neighbour pairs per rolled block and breaks ties on the rolled block
id, whereas oracle/topology.py (and the reference's plan.py / bridge_k.py)
work in ORIGINAL block ids with a (key - offset/64) mod nb tie-break. The two
agree only if the offsets, labels, scores and tie-breaks are all right, which
is what pins the table builder at grids the reference's tests do not reach.

Token identity is raster y*g + x.  Outputs are bool masks in raster identity
space [phase, query, key] (token level, for small grids) or block adjacency
in ORIGINAL image block ids [phase, nb, nb] (block level, any grid).
"""

from __future__ import annotations

import numpy as np


def _neighbor_pairs4(g):
    # Own enumeration (row-major, right then down); order does not matter here.
    ids = np.arange(g * g).reshape(g, g)
    right = np.stack((ids[:, :-1].ravel(), ids[:, 1:].ravel()), 1)
    down = np.stack((ids[:-1, :].ravel(), ids[1:, :].ravel()), 1)
    return np.concatenate((right, down))


def _setup(order, tile_count):
    order = np.asarray(order, dtype=np.int64)
    n = len(order)
    width = n // tile_count
    offsets = [0, width // 4, width // 2, 3 * width // 4]
    inverse = np.empty_like(order)
    inverse[order] = np.arange(n)
    labels = np.stack([((inverse - off) % n) // width for off in offsets])
    return order, inverse, labels, width, offsets


def _rolled_bridges(order, inverse, labels_p, offset, grid_size, block_size, count):
    """[(query_rolled_block, key_rolled_block)] chosen by the block_bridge rule (topology_oracle.py:308-328)."""
    n = len(order)
    pairs = _neighbor_pairs4(grid_size)
    block_ids = ((inverse - offset) % n) // block_size
    missing = pairs[labels_p[pairs[:, 0]] != labels_p[pairs[:, 1]]]
    nbr = n // block_size
    scores = np.zeros((nbr, nbr), dtype=np.int64)
    ba, bb = block_ids[missing[:, 0]], block_ids[missing[:, 1]]
    np.add.at(scores, (ba, bb), 1)
    np.add.at(scores, (bb, ba), 1)
    chosen = []
    for query in range(nbr):
        keys = np.nonzero(scores[query])[0]
        if len(keys) == 0:
            continue
        # sorted(choices, key=(-score, rolled key id))[:count]
        ranked = keys[np.lexsort((keys, -scores[query, keys]))][:count]
        chosen.extend((query, int(k)) for k in ranked)
    return chosen


def raster_masks(order, grid_size, tile_count, block_size, max_extra_blocks=0, shared_ids=None,
                 symmetric=False):
    """Token-level [4, n, n] masks: base | block_bridge extras (| shared rows/cols) (| transpose)."""
    order, inverse, labels, _, offsets = _setup(order, tile_count)
    n = len(order)
    masks = labels[:, :, None] == labels[:, None, :]
    if max_extra_blocks:
        for p, offset in enumerate(offsets):
            rolled = np.roll(order, -offset).reshape(-1, block_size)
            for q, k in _rolled_bridges(order, inverse, labels[p], offset, grid_size, block_size,
                                        max_extra_blocks):
                masks[p][np.ix_(rolled[q], rolled[k])] = True
    if shared_ids is not None:
        masks[:, shared_ids, :] = True
        masks[:, :, shared_ids] = True
    if symmetric:
        masks = masks | masks.transpose(0, 2, 1)
    assert masks.shape == (4, n, n)
    return masks


def block_adjacency(order, grid_size, tile_count, block_size, max_extra_blocks=0, symmetric=False):
    """Block-level [4, nb, nb] adjacency in ORIGINAL block ids (no shared region).

    Rolled block j of phase offset o holds original sequence positions
    j*bs + o .. (original block (j + o/bs) mod nb), because o is block aligned.
    """
    order, inverse, labels, width, offsets = _setup(order, tile_count)
    n = len(order)
    nb = n // block_size
    per_tile = width // block_size
    out = np.zeros((4, nb, nb), dtype=bool)
    for p, offset in enumerate(offsets):
        assert offset % block_size == 0
        tile_of_rolled = np.arange(nb) // per_tile
        adj_rolled = tile_of_rolled[:, None] == tile_of_rolled[None, :]
        if max_extra_blocks:
            for q, k in _rolled_bridges(order, inverse, labels[p], offset, grid_size, block_size,
                                        max_extra_blocks):
                adj_rolled[q, k] = True
        if symmetric:
            adj_rolled = adj_rolled | adj_rolled.T
        to_original = (np.arange(nb) + offset // block_size) % nb
        adj = np.zeros_like(adj_rolled)
        adj[np.ix_(to_original, to_original)] = adj_rolled
        out[p] = adj
    return out
