"""CPU: the host table builder (device="cpu", the *_host entry points) is bit-exact with the oracle.

The same drop-in calls as the GPU table tests (hilbert_order, build_plan, bridge_k_plan,
pair_metadata, paired_plan_device, pair_rows_device), run on a machine without a GPU, as the
reference's CPU-only suite runs them.  The attention kernels have no host path.
"""

import numpy as np
import pytest
import torch

from oracle import topology as T
from tests.helpers import eq_exact, oracle_paired, oracle_plan, plan_eq

CPU = "cpu"


@pytest.mark.parametrize("grid", [2, 4, 8, 16, 64, 128, 256])
def test_hilbert_order_host(grid):
    from hilberta_amd.geometry import hilbert_order

    eq_exact(hilbert_order(grid, device=CPU), T.hilbert_order(grid), f"hilbert {grid}")


@pytest.mark.parametrize("grid,block,text", [(16, 4, 16), (64, 64, 512), (128, 64, 512)])
@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("bridge", [False, True])
def test_build_plan_host(grid, block, text, tiles, shared, bridge):
    from hilberta_amd.plan import build_plan

    plan = build_plan(tiles, grid, text, shared, bridge, block, device=CPU)
    plan_eq(plan, T.build_plan(tiles, grid, text, shared, bridge, block), "build_plan", directed=True)


@pytest.mark.parametrize("grid", [64, 128, 256])
@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_bridge_k_plan_host(grid, tiles, k):
    from hilberta_amd.bridge_k import bridge_k_plan

    plan = bridge_k_plan(tiles, k, False, grid_size=grid, device=CPU)
    plan_eq(plan, T.bridge_k_plan(tiles, k, False, grid_size=grid), f"bridge_k g{grid} t{tiles} k{k}",
            directed=False)


@pytest.mark.parametrize("tiles", [4, 16])
def test_bridge_k_shared_host(tiles):
    from hilberta_amd.bridge_k import bridge_k_plan

    plan = bridge_k_plan(tiles, 2, True, grid_size=64, device=CPU)
    plan_eq(plan, T.bridge_k_plan(tiles, 2, True, grid_size=64), "bridge_k shared", directed=False)


def test_pair_metadata_hand_vector_host():
    """The reference test's hand vector (tests/test_paired_metadata.py:46-55): KV128 flags."""
    from hilberta_amd.paired_metadata import pair_metadata, unpair_metadata

    ids = torch.tensor([[0, 1, 2, 4], [0, 1, 3, 5], [0, 1, 4, 5], [0, 1, 4, 5]], dtype=torch.int32)
    counts = torch.full((4,), 4, dtype=torch.int32)
    meta = pair_metadata(ids, counts, tokens=384, global_tokens=128, key_block_size=128, device=CPU)
    assert meta.kv_indices[0, :3].tolist() == [0, 1, 2]
    assert meta.kv_flags[0, :3].tolist() == [15, 9, 9]
    assert unpair_metadata(meta) == ids.tolist()


@pytest.mark.parametrize("name", ["1024_t4k1", "1024_t16k3", "2048_t16k3", "4096_t16k3"])
@pytest.mark.parametrize("key_block", [64, 128])
def test_pair_metadata_host(name, key_block):
    from hilberta_amd.paired_metadata import pair_metadata

    plan = oracle_plan(name)
    for phase in range(4):
        p = plan["phases"][phase]
        ref = oracle_paired(plan, phase, key_block_size=key_block)
        meta = pair_metadata(torch.from_numpy(p["kv_indices"]), torch.from_numpy(p["kv_counts"]),
                             tokens=plan["total_tokens"], global_tokens=plan["global_tokens"],
                             key_block_size=key_block, device=CPU)
        for f in ("kv_indices", "kv_flags", "kv_counts"):
            eq_exact(getattr(meta, f), ref[f], f"{name} phase {phase} {f}")


@pytest.mark.parametrize("grid,tiles,k,shared,key_block", [
    (64, 4, 1, False, 64), (64, 16, 2, False, 64), (64, 4, 4, False, 128), (64, 16, 3, True, 64),
    (128, 4, 1, False, 64), (128, 16, 3, False, 64), (128, 16, 3, False, 128), (128, 4, 2, True, 64),
    (256, 16, 3, False, 64), (256, 4, 1, False, 64)])
def test_paired_plan_host(grid, tiles, k, shared, key_block):
    """paired_plan_device(device="cpu"): every layout array and the four phases' paired tables,
    widths and zero padding included, against bridge_k_plan + pair_metadata of the oracle."""
    from hilberta_amd.bridge_k import paired_plan_device

    dp = paired_plan_device(tiles, k, shared, grid_size=grid, key_block_size=key_block, device=CPU)
    ref_plan = T.bridge_k_plan(tiles, k, shared, grid_size=grid)
    for f in ("image_order", "inverse_image_order", "original_order", "physical_original_blocks"):
        eq_exact(getattr(dp.layout, f), ref_plan[f], f)
    assert dp.global_tokens == ref_plan["global_tokens"]
    for phase, meta in enumerate(dp.phases):
        ref = oracle_paired(ref_plan, phase, key_block_size=key_block)
        assert meta.tokens == ref_plan["total_tokens"]
        assert meta.global_tokens == ref_plan["global_tokens"]
        for f in ("kv_indices", "kv_flags", "kv_counts"):
            assert getattr(meta, f).device.type == "cpu" and getattr(meta, f).is_contiguous()
            eq_exact(getattr(meta, f), ref[f], f"host plan phase {phase} {f}")


@pytest.mark.parametrize("name,phase,kb", [("1024_t16k3", 0, 64), ("1024_t4k1", 1, 128),
                                           ("2048_t16k3", 2, 64), ("2048_t4k1", 1, 128)])
def test_pair_rows_host(name, phase, kb):
    """hb_pair_rows_host against pair_metadata, with garbage past each row's count."""
    from hilberta_amd._tables import pair_rows_device

    plan = oracle_plan(name)
    p = plan["phases"][phase]
    ref = oracle_paired(plan, phase, key_block_size=kb)
    ids_np, counts_np = np.asarray(p["kv_indices"]), np.asarray(p["kv_counts"])
    rows, width = ids_np.shape
    blocks = plan["total_tokens"] // 64
    pwidth = min(2 * width, -(-blocks // (kb // 64)))
    noisy = ids_np.copy()
    for r in range(rows):
        c = int(counts_np[r])
        if c < width:
            noisy[r, c:] = blocks + 7 if r % 2 else ids_np[r, 0]
    ids, flags, counts = pair_rows_device(torch.from_numpy(noisy), torch.from_numpy(counts_np),
                                          blocks, key_block_size=kb, paired_width=pwidth)
    ids, flags, counts = ids.numpy(), flags.numpy(), counts.numpy()
    rw = ref["kv_indices"].shape[1]
    assert np.array_equal(counts, ref["kv_counts"])
    assert np.array_equal(ids[:, :rw], ref["kv_indices"]) and np.array_equal(flags[:, :rw], ref["kv_flags"])
    assert not ids[:, rw:].any() and not flags[:, rw:].any()


@pytest.mark.parametrize("kb", [64, 128])
def test_pair_rows_host_odd_rows(kb):
    """An odd row count pairs from the end: paired row 0 holds the first row alone as half 1;
    paired rows r > 0 equal pair_metadata's rows of the even table it was cut from."""
    from hilberta_amd._tables import pair_rows_device

    plan = oracle_plan("1024_t16k3")
    p = plan["phases"][2]
    full = oracle_paired(plan, 2, key_block_size=kb)
    ids_np = np.ascontiguousarray(np.asarray(p["kv_indices"])[1:])
    counts_np = np.ascontiguousarray(np.asarray(p["kv_counts"])[1:])
    rows, width = ids_np.shape
    blocks = plan["total_tokens"] // 64
    pwidth = min(2 * width, -(-blocks // (kb // 64)))
    pid, pfl, pct = (x.numpy() for x in pair_rows_device(
        torch.from_numpy(ids_np), torch.from_numpy(counts_np), blocks, key_block_size=kb,
        paired_width=pwidth))
    assert pid.shape == ((rows + 1) // 2, pwidth)
    r = kb // 64
    exp0 = {}
    for b in ids_np[0, :counts_np[0]].tolist():
        exp0[b // r] = exp0.get(b // r, 0) | (1 << (1 + 2 * (b % r)))
    keys = sorted(exp0)
    assert pct[0] == len(keys)
    assert pid[0, :pct[0]].tolist() == keys and pfl[0, :pct[0]].tolist() == [exp0[b] for b in keys]
    rw = full["kv_indices"].shape[1]
    assert np.array_equal(pct[1:], full["kv_counts"][1:])
    assert np.array_equal(pid[1:, :rw], full["kv_indices"][1:])
    assert np.array_equal(pfl[1:, :rw], full["kv_flags"][1:])


def test_pair_rows_host_overflow_and_limits():
    """A width below the widest union cuts rows and sets the overflow word; the exact width leaves
    it clear.  The host accepts the tables the device accepts: at most 16384 key blocks."""
    from hilberta_amd._tables import pair_rows_device

    plan = oracle_plan("1024_t16k3")
    p = plan["phases"][1]
    ref = oracle_paired(plan, 1)
    exact = ref["kv_indices"].shape[1]
    ids = torch.from_numpy(np.asarray(p["kv_indices"]))
    counts = torch.from_numpy(np.asarray(p["kv_counts"]))
    blocks = plan["total_tokens"] // 64
    for width, expect in ((exact, 0), (exact - 1, 1), (4, 1)):
        flag = torch.zeros((), dtype=torch.int32)
        pid, _, pct = pair_rows_device(ids, counts, blocks, paired_width=width, overflow=flag)
        assert int(flag) == expect, width
        assert np.array_equal(pct.numpy(), np.minimum(ref["kv_counts"], width))
    with pytest.raises(ValueError, match="total_blocks"):
        pair_rows_device(ids, counts, 16385, paired_width=8)
    with pytest.raises(ValueError, match="int32"):
        pair_rows_device(ids.long(), counts, blocks, paired_width=8)


def test_host_builder_rejects_what_the_device_rejects():
    from hilberta_amd._tables import hilbert_order_device, layout_device, phase_bits_device
    from hilberta_amd.bridge_k import paired_plan_device

    with pytest.raises(ValueError, match="power of two"):
        hilbert_order_device(12, CPU)
    with pytest.raises(ValueError, match="power of two"):
        layout_device(24, 64, 512, False, CPU)
    layout = layout_device(64, 64, 512, False, CPU)
    with pytest.raises(ValueError, match="bridge K"):
        phase_bits_device(layout, 4, 0, 2, 5)
    with pytest.raises(ValueError, match="phase"):
        phase_bits_device(layout, 4, 4, 0, 1)
    with pytest.raises(ValueError, match="block aligned"):
        phase_bits_device(layout, 64, 0, 0, 1)
    with pytest.raises(ValueError, match="KV must be 64/128"):
        paired_plan_device(4, 1, grid_size=64, key_block_size=96, device=CPU)
    with pytest.raises(ValueError, match="host"):
        hilbert_order_device(8, "meta")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the GPU-less default")
def test_default_device_without_gpu_names_the_host_builder():
    """Without a GPU the default device raises and names device='cpu'; the host builder is never
    chosen silently in place of a GPU."""
    from hilberta_amd.geometry import hilbert_order

    with pytest.raises(RuntimeError, match="device='cpu'"):
        hilbert_order(8)


@pytest.mark.parametrize("seed", range(12))
def test_pair_metadata_host_random_tables(seed):
    """Random valid tables (global prefix, unique ids in any order, ragged counts, garbage past
    each count) on random geometries: pair_metadata(device="cpu") and hb_pair_rows_host both
    equal the oracle's pair_metadata, at 64- and 128-token key blocks."""
    from hilberta_amd._tables import pair_rows_device
    from hilberta_amd.paired_metadata import pair_metadata

    rng = np.random.default_rng(seed)
    G = 128 * int(rng.integers(0, 5))
    rows = 2 * int(rng.integers(1, 40))
    N = G + 64 * rows
    T_ = N // 64
    width = G // 64 + int(rng.integers(1, 24))
    ids = np.full((rows, width), -1, np.int32)
    counts = np.zeros(rows, np.int32)
    for r in range(rows):
        extra = rng.choice(np.arange(G // 64, T_), size=int(rng.integers(1, min(width - G // 64, T_ - G // 64) + 1)),
                           replace=False)
        row = np.concatenate([np.arange(G // 64), extra]).astype(np.int32)
        rng.shuffle(row)
        ids[r, :len(row)] = row
        ids[r, len(row):] = rng.integers(0, T_, size=width - len(row))
        counts[r] = len(row)
    for kb in (64, 128):
        ref = T.pair_metadata(ids, counts, tokens=N, global_tokens=G, key_block_size=kb)
        meta = pair_metadata(torch.from_numpy(ids), torch.from_numpy(counts), tokens=N,
                             global_tokens=G, key_block_size=kb, device=CPU)
        for f in ("kv_indices", "kv_flags", "kv_counts"):
            eq_exact(getattr(meta, f), ref[f], f"seed {seed} KB{kb} {f}")
        w = ref["kv_indices"].shape[1]
        pid, pfl, pct = pair_rows_device(torch.from_numpy(ids), torch.from_numpy(counts), T_,
                                         key_block_size=kb, paired_width=w)
        eq_exact(pid, ref["kv_indices"], "pair_rows ids")
        eq_exact(pfl, ref["kv_flags"], "pair_rows flags")
        eq_exact(pct, ref["kv_counts"], "pair_rows counts")
