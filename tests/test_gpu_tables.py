"""GPU: the HIP table builder and permutation gather are bit-exact against the CPU oracle / torch."""

import numpy as np
import pytest
import torch

from oracle import topology as T
from tests.helpers import eq_exact as _eq, oracle_paired, oracle_plan, plan_eq as _plan_eq, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("grid", [2, 4, 8, 64, 128, 256])
def test_hilbert_order(hip_device, grid):
    from hilberta_amd.geometry import hilbert_order

    _eq(hilbert_order(grid, device=hip_device), T.hilbert_order(grid), f"hilbert {grid}")


@pytest.mark.parametrize("grid,block,text", [(16, 4, 16), (64, 64, 512)])
@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("bridge", [False, True])
def test_build_plan_bit_exact(hip_device, grid, block, text, tiles, shared, bridge):
    from hilberta_amd.plan import build_plan

    say(f"case build_plan grid={grid} block={block} tiles={tiles} shared={shared} bridge={bridge}")
    dev = build_plan(tiles, grid, text, shared, bridge, block, device=hip_device)
    ref = T.build_plan(tiles, grid, text, shared, bridge, block)
    _plan_eq(dev, ref, "build_plan", directed=True)


@pytest.mark.parametrize("grid", [64, 128, 256])
@pytest.mark.parametrize("tiles", [4, 16])
@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_bridge_k_plan_bit_exact(hip_device, grid, tiles, k):
    from hilberta_amd.bridge_k import bridge_k_plan

    say(f"case bridge_k grid={grid} tiles={tiles} k={k}")
    dev = bridge_k_plan(tiles, k, False, grid_size=grid, device=hip_device)
    ref = T.bridge_k_plan(tiles, k, False, grid_size=grid)
    _plan_eq(dev, ref, f"bridge_k g{grid} t{tiles} k{k}", directed=False)


@pytest.mark.parametrize("tiles", [4, 16])
def test_bridge_k_shared_bit_exact(hip_device, tiles):
    from hilberta_amd.bridge_k import bridge_k_plan

    dev = bridge_k_plan(tiles, 2, True, grid_size=64, device=hip_device)
    ref = T.bridge_k_plan(tiles, 2, True, grid_size=64)
    _plan_eq(dev, ref, "bridge_k shared", directed=False)


def test_pair_metadata_hand_vector(hip_device):
    from hilberta_amd.paired_metadata import pair_metadata, unpair_metadata

    ids = torch.tensor([[0, 1, 2, 4], [0, 1, 3, 5], [0, 1, 4, 5], [0, 1, 4, 5]], dtype=torch.int32)
    counts = torch.full((4,), 4, dtype=torch.int32)
    meta = pair_metadata(ids, counts, tokens=384, global_tokens=128, key_block_size=128,
                         device=hip_device)
    assert meta.kv_indices[0, :3].tolist() == [0, 1, 2]
    assert meta.kv_flags[0, :3].tolist() == [15, 9, 9]
    assert unpair_metadata(meta) == ids.tolist()


@pytest.mark.parametrize("name,grid,tiles,k", [("1024_t4k1", 64, 4, 1), ("1024_t16k3", 64, 16, 3),
                                               ("2048_t16k3", 128, 16, 3), ("4096_t16k3", 256, 16, 3)])
@pytest.mark.parametrize("key_block", [64, 128])
def test_pair_metadata_bit_exact(hip_device, name, grid, tiles, k, key_block):
    from hilberta_amd.paired_metadata import pair_metadata

    ref_plan = T.bridge_k_plan(tiles, k, False, grid_size=grid)
    for phase in range(4):
        say(f"case pair_metadata {name} phase {phase} KB{key_block}")
        p = ref_plan["phases"][phase]
        ref = T.pair_metadata(p["kv_indices"], p["kv_counts"], tokens=ref_plan["total_tokens"],
                              global_tokens=ref_plan["global_tokens"], key_block_size=key_block)
        meta = pair_metadata(torch.from_numpy(p["kv_indices"]), torch.from_numpy(p["kv_counts"]),
                             tokens=ref_plan["total_tokens"], global_tokens=ref_plan["global_tokens"],
                             key_block_size=key_block, device=hip_device)
        for f in ("kv_indices", "kv_flags", "kv_counts"):
            _eq(getattr(meta, f), ref[f], f"{name} phase {phase} {f}")


@pytest.mark.parametrize("grid,tiles,k,shared,key_block", [
    (64, 4, 1, False, 64), (64, 16, 2, False, 64), (64, 4, 4, False, 128), (64, 16, 3, True, 64),
    (128, 4, 1, False, 64), (128, 16, 3, False, 64), (128, 16, 3, False, 128), (128, 4, 2, True, 64),
    (256, 16, 3, False, 64), (256, 4, 1, False, 64)])
def test_paired_plan_device_bit_exact(hip_device, grid, tiles, k, shared, key_block):
    """The fused device plan (six launches, one host read) against the oracle: every layout array
    and the four phases' paired tables, widths and zero padding included."""
    from hilberta_amd.bridge_k import paired_plan_device

    say(f"case paired_plan_device grid={grid} tiles={tiles} K={k} shared={shared} KB{key_block}")
    dp = paired_plan_device(tiles, k, shared, grid_size=grid, key_block_size=key_block,
                            device=hip_device)
    ref_plan = T.bridge_k_plan(tiles, k, shared, grid_size=grid)
    for f in ("image_order", "inverse_image_order", "original_order", "physical_original_blocks"):
        _eq(getattr(dp.layout, f), ref_plan[f], f)
    assert dp.global_tokens == ref_plan["global_tokens"]
    for phase, meta in enumerate(dp.phases):
        p = ref_plan["phases"][phase]
        ref = T.pair_metadata(p["kv_indices"], p["kv_counts"], tokens=ref_plan["total_tokens"],
                              global_tokens=ref_plan["global_tokens"], key_block_size=key_block)
        assert meta.tokens == ref_plan["total_tokens"]
        assert meta.global_tokens == ref_plan["global_tokens"]
        for f in ("kv_indices", "kv_flags", "kv_counts"):
            assert getattr(meta, f).is_contiguous()
            _eq(getattr(meta, f), ref[f], f"device plan phase {phase} {f}")


# ---------------------------------------------------------------------------- permutation
@pytest.mark.parametrize(
    "shape,dim,dtype",
    [
        ((1, 4096, 64), 1, torch.bfloat16),  # 1024 px latents
        ((2, 16384, 64), 1, torch.bfloat16),  # 2048 px latents, B=2
        ((4096, 3), 0, torch.float32),  # position ids (12-byte rows)
        ((2, 4096, 3), 1, torch.int64),  # batched ids (24-byte rows)
        ((1, 4608, 3072), 1, torch.bfloat16),  # hidden states
        ((1, 4608, 24, 128), 1, torch.bfloat16),  # BNHD projections
        ((3, 1000, 7), 1, torch.uint8),  # odd byte rows
    ],
)
def test_index_select_rows_bit_exact(hip_device, shape, dim, dtype):
    from hilberta_amd.layout import index_select_rows

    gen = torch.Generator("cpu").manual_seed(7)
    if dtype.is_floating_point:
        x = torch.randn(shape, generator=gen).to(dtype)
    else:
        x = torch.randint(0, 100, shape, generator=gen).to(dtype)
    x = x.to(hip_device)
    index = torch.randperm(shape[dim], generator=gen).to(hip_device)
    out = index_select_rows(x, dim, index)
    assert torch.equal(out, x.index_select(dim, index))
    inv = torch.empty_like(index)
    inv[index] = torch.arange(len(index), device=hip_device)
    assert torch.equal(index_select_rows(out, dim, inv), x)  # unpermute round trip


def test_index_select_rows_strided_and_errors(hip_device):
    from hilberta_amd.layout import index_select_rows

    x = torch.randn(2, 512, 24, 128, device=hip_device).to(torch.bfloat16)
    view = x.transpose(1, 2)[:, :, :, :]  # [2, 24, 512, 128], gather along the token dim 2
    index = torch.randperm(512, device=hip_device)
    assert torch.equal(index_select_rows(view, 2, index), view.index_select(2, index))
    err = torch.zeros((), dtype=torch.int32, device=hip_device)
    bad = index.clone()
    bad[5] = 512
    index_select_rows(x, 1, bad, error=err)
    assert int(err) == 1
    with pytest.raises(ValueError):
        index_select_rows(x.transpose(2, 3), 1, index)  # row not contiguous


def test_index_select_rows_out_of_range_contract(hip_device):
    """check=True raises as index_select does (flux_adapter.py:209-212); the default trusts the
    index (plan orders are checked once at build), skips an out-of-range row, and writes every
    in-range row exactly as index_select would."""
    from hilberta_amd.layout import index_select_rows

    x = torch.randn(2, 512, 64, device=hip_device).to(torch.bfloat16)
    index = torch.randperm(512, device=hip_device)
    assert torch.equal(index_select_rows(x, 1, index, check=True), x.index_select(1, index))
    for bad_value in (512, -1, 1 << 40):
        bad = index.clone()
        bad[7] = bad_value
        with pytest.raises(IndexError, match="out of range"):
            index_select_rows(x, 1, bad, check=True)
        out = torch.full((2, 512, 64), 3.0, device=hip_device).to(torch.bfloat16)
        index_select_rows(x, 1, bad, out=out)
        keep = torch.ones(512, dtype=torch.bool, device=hip_device)
        keep[7] = False
        assert torch.equal(out[:, keep], x.index_select(1, index[keep]))
        assert torch.equal(out[:, 7], torch.full_like(out[:, 7], 3.0))  # left unwritten


@pytest.mark.parametrize("grid,tiles,shared", [(64, 4, False), (128, 16, False), (64, 16, True)])
def test_plan_orders_are_checked_permutations(hip_device, grid, tiles, shared):
    """The layout builder's orders (validated on the device at build time) are inverse
    permutations, so the per-forward gathers may trust them."""
    from hilberta_amd._tables import layout_device

    lay = layout_device(grid, 64, 512, shared, device=hip_device)
    n = grid * grid
    ar = torch.arange(n, device=hip_device)
    assert torch.equal(torch.sort(lay.image_order).values, ar)
    assert torch.equal(lay.inverse_image_order[lay.image_order], ar)


def test_plan_layout_permutes_latents(hip_device):
    """Permute at entry, unpermute at exit with the device plan's orders (sampling_layout.py:88-116)."""
    from hilberta_amd.bridge_k import paired_plan_device
    from hilberta_amd.layout import permute_tokens, unpermute_tokens

    dp = paired_plan_device(16, 3, grid_size=128, device=hip_device)
    lat = torch.randn(1, 16384, 64, device=hip_device).to(torch.bfloat16)
    packed = permute_tokens(lat, dp.layout.image_order)
    assert torch.equal(packed, lat.index_select(1, dp.layout.image_order))
    assert torch.equal(unpermute_tokens(packed, dp.layout.inverse_image_order), lat)


@pytest.mark.parametrize("name,phase,kb", [("1024_t16k3", 0, 64), ("1024_t16k3", 3, 64),
                                           ("1024_t4k1", 1, 128), ("2048_t16k3", 2, 64),
                                           ("2048_t4k1", 1, 128)])
def test_pair_rows_equals_pair_metadata(hip_device, name, phase, kb):
    """hb_pair_rows (one launch, padded width, no host sync) is bit-exact with pair_metadata."""
    from hilberta_amd._tables import pair_rows_device

    plan = oracle_plan(name)
    p = plan["phases"][phase]
    ref = oracle_paired(plan, phase, key_block_size=kb)
    ids_np, counts_np = np.asarray(p["kv_indices"]), np.asarray(p["kv_counts"])
    rows, width = ids_np.shape
    blocks = plan["total_tokens"] // 64
    pwidth = min(2 * width, -(-blocks // (kb // 64)))
    # entries past each row's count hold garbage (an out-of-range id and a duplicate): ignored
    noisy = ids_np.copy()
    for r in range(rows):
        c = int(counts_np[r])
        if c < width:
            noisy[r, c:] = blocks + 7 if r % 2 else ids_np[r, 0]
    say(f"case pair_rows {name} phase {phase} KB{kb} width {pwidth}")
    ids, flags, counts = pair_rows_device(torch.from_numpy(noisy).to(hip_device),
                                          torch.from_numpy(counts_np).to(hip_device), blocks,
                                          key_block_size=kb, paired_width=pwidth)
    torch.cuda.synchronize()
    ids, flags, counts = ids.cpu().numpy(), flags.cpu().numpy(), counts.cpu().numpy()
    ref_ids, ref_flags, ref_counts = (np.asarray(ref[k]) for k in ("kv_indices", "kv_flags", "kv_counts"))
    assert np.array_equal(counts, ref_counts)
    rw = ref_ids.shape[1]
    assert rw <= pwidth
    assert np.array_equal(ids[:, :rw], ref_ids) and np.array_equal(flags[:, :rw], ref_flags)
    assert not ids[:, rw:].any() and not flags[:, rw:].any()


@pytest.mark.parametrize("kb", [64, 128])
def test_pair_rows_odd_row_count(hip_device, kb):
    """An odd row count is paired from the end.  Rows 1..63 of a 64-row table: paired row 0 holds
    row 1 alone as half 1 (an empty half 0, so flag bits 2 + 8 * key_half only), and paired rows
    r > 0 hold rows 2r and 2r + 1 of the full table, bit-exact with pair_metadata's rows r > 0."""
    from hilberta_amd._tables import pair_rows_device

    plan = oracle_plan("1024_t16k3")
    p = plan["phases"][2]
    full = oracle_paired(plan, 2, key_block_size=kb)
    ids_np = np.ascontiguousarray(np.asarray(p["kv_indices"])[1:])
    counts_np = np.ascontiguousarray(np.asarray(p["kv_counts"])[1:])
    rows, width = ids_np.shape
    blocks = plan["total_tokens"] // 64
    pwidth = min(2 * width, -(-blocks // (kb // 64)))
    say(f"case pair_rows odd rows={rows} KB{kb}")
    pid, pfl, pct = pair_rows_device(torch.from_numpy(ids_np).to(hip_device),
                                     torch.from_numpy(counts_np).to(hip_device), blocks,
                                     key_block_size=kb, paired_width=pwidth)
    torch.cuda.synchronize()
    pid, pfl, pct = pid.cpu().numpy(), pfl.cpu().numpy(), pct.cpu().numpy()
    assert pid.shape == ((rows + 1) // 2, pwidth)
    # paired row 0: the first remaining row alone, as half 1
    r = kb // 64
    exp0 = {}
    for b in ids_np[0, :counts_np[0]].tolist():
        exp0[b // r] = exp0.get(b // r, 0) | (1 << (1 + 2 * (b % r)))
    keys = sorted(exp0)
    assert pct[0] == len(keys)
    assert pid[0, :pct[0]].tolist() == keys and pfl[0, :pct[0]].tolist() == [exp0[b] for b in keys]
    assert not pid[0, pct[0]:].any() and not pfl[0, pct[0]:].any()
    ref_ids, ref_flags, ref_counts = (np.asarray(full[k])[1:] for k in ("kv_indices", "kv_flags", "kv_counts"))
    rw = ref_ids.shape[1]
    assert np.array_equal(pct[1:], ref_counts)
    assert np.array_equal(pid[1:, :rw], ref_ids) and np.array_equal(pfl[1:, :rw], ref_flags)
    assert not pid[1:, rw:].any() and not pfl[1:, rw:].any()


def test_pair_rows_reports_overflow(hip_device):
    """A paired width below the widest union cuts those rows to the width and raises the
    overflow word; the exact width (the widest union of pair_metadata) leaves it at zero."""
    from hilberta_amd._tables import pair_rows_device

    plan = oracle_plan("1024_t16k3")
    p = plan["phases"][1]
    ref = oracle_paired(plan, 1)
    exact = ref["kv_indices"].shape[1]
    ids = torch.from_numpy(np.asarray(p["kv_indices"])).to(hip_device)
    counts = torch.from_numpy(np.asarray(p["kv_counts"])).to(hip_device)
    blocks = plan["total_tokens"] // 64
    for width, expect in ((exact, 0), (exact - 1, 1), (4, 1)):
        say(f"case pair_rows overflow width {width}")
        flag = torch.zeros((), dtype=torch.int32, device=hip_device)
        pid, _, pct = pair_rows_device(ids, counts, blocks, paired_width=width, overflow=flag)
        torch.cuda.synchronize()
        assert int(flag) == expect, width
        ref_counts = np.asarray(ref["kv_counts"])
        assert np.array_equal(pct.cpu().numpy(), np.minimum(ref_counts, width))
        assert np.array_equal(pid.cpu().numpy()[:, :width][ref_counts >= width],
                              np.asarray(ref["kv_indices"])[ref_counts >= width, :width])


def test_pair_rows_beyond_2048_key_blocks(hip_device):
    """Tables of more than 2048 key blocks pair on the device too (up to 16384): random rows over
    4008 key blocks, bit-exact with pair_metadata."""
    from hilberta_amd._tables import pair_rows_device

    G, rows = 512, 4000
    N = G + 64 * rows
    T_ = N // 64
    rng = np.random.default_rng(17)
    width = G // 64 + 10
    ids = np.zeros((rows, width), np.int32)
    counts = np.zeros(rows, np.int32)
    for r in range(rows):
        extra = rng.choice(np.arange(G // 64, T_), size=rng.integers(1, 11), replace=False)
        row = np.concatenate([np.arange(G // 64), np.sort(extra)]).astype(np.int32)
        ids[r, :len(row)] = row
        counts[r] = len(row)
    ref = T.pair_metadata(ids, counts, tokens=N, global_tokens=G)
    say(f"case pair_rows T={T_}")
    pid, pfl, pct = pair_rows_device(torch.from_numpy(ids).to(hip_device),
                                     torch.from_numpy(counts).to(hip_device), T_,
                                     paired_width=2 * width)
    torch.cuda.synchronize()
    pid, pfl, pct = pid.cpu().numpy(), pfl.cpu().numpy(), pct.cpu().numpy()
    rw = ref["kv_indices"].shape[1]
    assert np.array_equal(pct, ref["kv_counts"])
    assert np.array_equal(pid[:, :rw], ref["kv_indices"]) and np.array_equal(pfl[:, :rw], ref["kv_flags"])
    assert not pid[:, rw:].any() and not pfl[:, rw:].any()


@pytest.mark.parametrize("grid,tiles,k,shared,key_block,text", [
    (128, 16, 3, True, 128, 512), (256, 16, 4, True, 64, 512), (512, 16, 3, False, 64, 512),
    (64, 16, 2, False, 64, 256), (128, 4, 4, True, 128, 1024), (256, 64, 1, False, 128, 128)])
def test_host_and_device_builders_agree(hip_device, grid, tiles, k, shared, key_block, text):
    """The host builder (device="cpu") and the fused device plan write the same layout and paired
    tables bit for bit, up to 8192 px (4096 image blocks), beyond the oracle-checked sizes; and
    the same unpaired tables through build_plan / bridge_k_plan."""
    from hilberta_amd.bridge_k import bridge_k_plan, paired_plan_device

    say(f"case host==device grid={grid} tiles={tiles} K={k} shared={shared} KB{key_block} text={text}")
    dev = paired_plan_device(tiles, k, shared, grid_size=grid, text_tokens=text,
                             key_block_size=key_block, device=hip_device)
    host = paired_plan_device(tiles, k, shared, grid_size=grid, text_tokens=text,
                              key_block_size=key_block, device="cpu")
    for f in ("original_order", "inverse_original", "image_order", "inverse_image_order",
              "physical_original_blocks", "original_to_physical"):
        _eq(getattr(dev.layout, f), getattr(host.layout, f).numpy(), f)
    for phase, (d, h) in enumerate(zip(dev.phases, host.phases)):
        for f in ("kv_indices", "kv_flags", "kv_counts"):
            _eq(getattr(d, f), getattr(h, f).numpy(), f"phase {phase} {f}")
    if grid <= 256 and text == 512:  # bridge_k_plan has the reference's fixed 512-token prefix
        d = bridge_k_plan(tiles, k, shared, grid_size=grid, device=hip_device)
        h = bridge_k_plan(tiles, k, shared, grid_size=grid, device="cpu")
        for pd, ph in zip(d.phases, h.phases):
            _eq(pd.kv_indices, ph.kv_indices.numpy(), "bridge_k kv_indices")
            _eq(pd.bridge_original_blocks, ph.bridge_original_blocks.numpy(), "bridges")


@pytest.mark.parametrize("rows,kb", [(4001, 64), (4000, 128)])
def test_host_and_device_pair_rows_agree(hip_device, rows, kb):
    """hb_pair_rows and hb_pair_rows_host on random ragged tables over ~4000 key blocks (odd and
    even row counts), garbage past each count included: identical ids, flags, counts and overflow."""
    from hilberta_amd._tables import pair_rows_device

    rng = np.random.default_rng(rows + kb)
    T_ = rows + 8
    width = 24
    ids = rng.integers(-3, T_ + 3, size=(rows, width), dtype=np.int32)
    counts = rng.integers(0, width + 3, size=rows, dtype=np.int32)
    say(f"case pair_rows host==device rows={rows} KB{kb}")
    for pwidth in (2 * width, 9):
        outs = []
        for device in (hip_device, torch.device("cpu")):
            flag = torch.zeros((), dtype=torch.int32, device=device)
            got = pair_rows_device(torch.from_numpy(ids).to(device), torch.from_numpy(counts).to(device),
                                   T_, key_block_size=kb, paired_width=pwidth, overflow=flag)
            outs.append([x.cpu().numpy() for x in got] + [int(flag)])
        for a, b, what in zip(outs[0], outs[1], ("ids", "flags", "counts", "overflow")):
            assert np.array_equal(a, b), f"{what} differ at width {pwidth}"
