"""Pins the CPU table oracle (oracle/topology.py) -- no GPU needed.

Mirrors the reference's CPU topology tests (tests/test_plan.py, tests/test_bridge_k.py,
tests/test_paired_metadata.py) and adds a second-algorithm check at the 2048/4096 grids.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import mask_oracle as M
from oracle import topology as T

GOLDEN = Path(__file__).resolve().parent / "golden"
KNOWN = json.loads((GOLDEN / "known_answers.json").read_text())


def _center_ids(grid):
    lo, hi = 3 * grid // 8, 5 * grid // 8
    return np.arange(grid * grid).reshape(grid, grid)[lo:hi, lo:hi].ravel()


# ------------------------------------------------------------------ geometry
def test_hilbert_hand_case():
    assert T.hilbert_order(2).tolist() == KNOWN["hilbert_grid2"]["order"]


@pytest.mark.parametrize("grid", [2, 4, 8, 64, 256])
def test_hilbert_is_a_local_permutation(grid):
    h = T.hilbert_order(grid)
    assert np.array_equal(np.sort(h), np.arange(grid * grid))
    y, x = h // grid, h % grid
    step = np.abs(np.diff(y)) + np.abs(np.diff(x))
    assert (step == 1).all()  # consecutive curve points are 4-neighbours


def test_hilbert_rejects_bad_grid():
    for g in (0, 1, 3, 12):
        with pytest.raises(ValueError):
            T.hilbert_order(g)


@pytest.mark.parametrize("grid", [1, 2, 5, 64])
def test_neighbor_pairs(grid):
    p4 = T.neighbor_pairs(grid, 4)
    assert len(p4) == 2 * grid * (grid - 1)
    assert (p4[:, 0] < p4[:, 1]).all()
    d = p4[:, 1] - p4[:, 0]
    assert set(d.tolist()) <= {1, grid}
    assert len({tuple(x) for x in p4.tolist()}) == len(p4)
    p8 = T.neighbor_pairs(grid, 8)
    assert len(p8) == 2 * grid * (grid - 1) + 2 * (grid - 1) ** 2
    if grid == 2:  # row-major, right then down then diagonals
        assert p8.tolist() == [[0, 1], [0, 2], [0, 3], [1, 3], [1, 2], [2, 3]]


# ------------------------------------------------------------------ build_plan
def test_known_bridge_budget_and_shared_layout():
    kb = KNOWN["build_plan_bridge_budget"]
    for tiles, expected in [(4, kb["tiles4"]), (16, kb["tiles16"])]:
        a, b = T.build_plan(tiles, bridge=False), T.build_plan(tiles)
        delta = [int((T.block_adjacency(b, i) & ~T.block_adjacency(a, i)).sum()) for i in range(4)]
        assert delta == expected
        assert a["physical_original_blocks"][:4].tolist() == kb["physical_original_blocks_head"]


@pytest.mark.parametrize("grid,block,text", [(16, 4, 16), (64, 64, 512)])
@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("bridge", [False, True])
def test_build_plan_equals_rolled_oracle(grid, block, text, tiles, shared, bridge):
    """Reference tests/test_plan.py:10-52 semantics, second algorithm in raster identity space."""
    p = T.build_plan(tiles, grid, text, shared, bridge, block)
    oracle = M.raster_masks(
        p["original_order"], grid, tiles, block, max_extra_blocks=1 if bridge else 0,
        shared_ids=_center_ids(grid) if shared else None,
    )
    order = p["image_order"]
    for phase in range(4):
        mask = T.dense_mask(p, phase)
        assert mask[:text].all() and mask[:, :text].all()
        assert np.array_equal(mask[text:, text:], oracle[phase][np.ix_(order, order)])
    assert np.array_equal(order[p["inverse_image_order"]], np.arange(grid**2))


def test_full_layout_gate():
    p = T.full_attention_plan(T.build_plan(16, 16, 16, True, True, 4))
    assert all(T.dense_mask(p, i).all() for i in range(4))


def test_unaligned_rejected():
    with pytest.raises(ValueError):
        T.build_plan(16, block_size=128)
    with pytest.raises(ValueError):
        T.build_plan(text_tokens=17)
    with pytest.raises(ValueError):
        T.build_plan(grid_size=48)


# ------------------------------------------------------------------ bridge_k_plan
@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("shared", [False, True])
def test_bridge_k1_is_symmetrised_build_plan(tiles, shared):
    """Reference tests/test_bridge_k.py:9-27 (K1 part)."""
    old = T.build_plan(tiles, shared=shared)
    new = T.bridge_k_plan(tiles, 1, shared)
    for i in range(4):
        a = T.block_adjacency(old, i)
        g = old["global_tokens"] // 64
        img = a[g:, g:] | a[g:, g:].T
        assert np.array_equal(T.block_adjacency(new, i)[g:, g:], img)


def test_bridge_k1_matches_reference_demo_data():
    demo = json.loads((GOLDEN / "demo_t4k1_grid64.json").read_text())
    p = T.bridge_k_plan(4, 1, False, grid_size=64)
    n, width = 4096, 1024
    for ph, ref in zip(p["phases"], demo["phases"]):
        assert ph["offset"] == ref["offset"]
        labels = [((b * 64 - ph["offset"]) % n) // width for b in range(64)]
        assert labels == ref["labels"]
        chosen = ph["bridge_original_blocks"][:, 0]
        edges = sorted({tuple(sorted((q, int(c)))) for q, c in enumerate(chosen) if c >= 0})
        assert edges == [tuple(e) for e in ref["edges"]]
        # every chosen bridge appears in both directions of the tables
        adj = T.block_adjacency(p, ph["offset"] // 256)
        for u, v in edges:
            assert adj[8 + u, 8 + v] and adj[8 + v, 8 + u]


@pytest.mark.parametrize("grid", [64, 128, 256])
@pytest.mark.parametrize("tiles", [4, 16])
def test_bridge_k_equals_second_algorithm(grid, tiles):
    """K1..K4 reciprocal tables vs rolled-coordinate block_bridge (topology_oracle.py:308-329 | T)."""
    previous = None
    for k in (1, 2, 3, 4):
        p = T.bridge_k_plan(tiles, k, False, grid_size=grid)
        other = M.block_adjacency(p["original_order"], grid, tiles, 64, max_extra_blocks=k,
                                  symmetric=True)
        g = p["global_tokens"] // 64
        current = np.stack([T.block_adjacency(p, i) for i in range(4)])
        assert np.array_equal(current[:, g:, g:], other)
        assert np.array_equal(current[:, g:, g:], current[:, g:, g:].transpose(0, 2, 1))
        assert current[:, :g].all() and current[:, :, :g].all()
        assert not current[:, g:, g:].all(-1).any()
        if previous is not None:
            assert not (previous & ~current).any()  # monotone in K
        previous = current


def test_bridge_k_shared_k2_oracle():
    """Reference tests/test_bridge_k.py:15-27 (K2 with and without the shared square), token level."""
    for tiles in (4, 16):
        for shared in (False, True):
            p = T.bridge_k_plan(tiles, 2, shared)
            oracle = M.raster_masks(p["original_order"], 64, tiles, 64, max_extra_blocks=2,
                                    shared_ids=p["image_order"][: p["shared_tokens"]] if shared else None,
                                    symmetric=True)
            text, inv = p["text_tokens"], p["inverse_image_order"]
            for i in range(4):
                actual = T.dense_mask(p, i)[text:, text:][np.ix_(inv, inv)]
                assert np.array_equal(actual, oracle[i])


def test_bad_k():
    for k in (0, 5, True):
        with pytest.raises(ValueError):
            T.bridge_k_plan(16, k)


# ------------------------------------------------------------------ pair_metadata
def test_paired_hand_vector():
    hv = KNOWN["paired_hand_vector"]
    ids = np.array(hv["kv_indices"], dtype=np.int32)
    counts = np.array(hv["kv_counts"], dtype=np.int32)
    meta = T.pair_metadata(ids, counts, tokens=hv["tokens"], global_tokens=hv["global_tokens"],
                           key_block_size=hv["key_block_size"])
    assert meta["kv_indices"][0, :3].tolist() == hv["expect_indices_row0_head3"]
    assert meta["kv_flags"][0, :3].tolist() == hv["expect_flags_row0_head3"]
    assert T.unpair_metadata(meta) == ids.tolist()


@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("bridge", [False, True])
def test_pair_round_trip_and_popcount(tiles, shared, bridge):
    """Reference tests/test_paired_metadata.py:10-44."""
    plan = T.build_plan(tiles, shared=shared, bridge=bridge)
    for phase in plan["phases"]:
        expected = [r[: int(n)].tolist() for r, n in zip(phase["kv_indices"], phase["kv_counts"])]
        for size in (64, 128):
            meta = T.pair_metadata(phase["kv_indices"], phase["kv_counts"],
                                   tokens=plan["total_tokens"], global_tokens=plan["global_tokens"],
                                   key_block_size=size)
            assert T.unpair_metadata(meta) == expected
            live = sum(int(f).bit_count() for r, n in zip(meta["kv_flags"], meta["kv_counts"])
                       for f in r[: int(n)])
            assert live == int(phase["kv_counts"].sum())
            # zero padding beyond each count, sorted unique ids
            for r, f, n in zip(meta["kv_indices"], meta["kv_flags"], meta["kv_counts"]):
                assert (r[n:] == 0).all() and (f[n:] == 0).all()
                assert (np.diff(r[:n]) > 0).all()


def test_validate_metadata_rejections():
    ids = np.array([[0, 1], [0, 2]], dtype=np.int32)
    counts = np.array([2, 2], dtype=np.int32)
    info = T.validate_metadata(ids, counts, tokens=192, global_tokens=64)
    assert info["total_directed_entries"] == 64 * 192 + 4 * 4096
    with pytest.raises(ValueError):
        T.validate_metadata(np.array([[0, 0], [0, 2]], np.int32), counts, tokens=192, global_tokens=64)
    with pytest.raises(ValueError):
        T.validate_metadata(np.array([[1, 2], [0, 2]], np.int32), counts, tokens=192, global_tokens=64)
    with pytest.raises(TypeError):
        T.validate_metadata(ids.astype(np.int64), counts, tokens=192, global_tokens=64)
