"""Randomised shapes and tables through paired_attention and sparse_attention.

Each case draws, from its own seed: batch 1-3, heads 1-5, head dim 64 or 128, bf16 or fp16, a
global prefix of 0-512 tokens (multiples of 128, so every table pairs), 2-16 paired rows, 64- or
128-key paired blocks, BHND or BNHD storage, the persistent grid size (default, or a handful of
workgroups so each crosses many items), and unpaired 64-query tables of 1-12 random blocks.  With
the global prefix on every row they are paired on the host by the oracle for paired_attention;
with the prefix dropped on some rows (or none, or all) they go as they are to sparse_attention,
which pairs them on the device.  A second set draws global prefixes of any multiple of 64 and
odd or even row counts, which sparse_attention pairs from the end with an overhanging half.

The reference applies every entry's flags (paired_kernel.py:70-84) and lets global query rows see
every key (paired_kernel.py:173-178); the oracle is fp32 dense masked attention on the CPU over
the paired-flag mask or the unpaired explicit mask (oracle/attention.py), at the tolerance of the
other parity tests.
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import topology as T
from tests.helpers import compare, device_paired, say

pytestmark = pytest.mark.gpu

CASES = 48


def _draw(case):
    rng = np.random.default_rng(9100 + case)
    c = {
        "B": int(rng.integers(1, 4)),
        "H": int(rng.integers(1, 6)),
        "D": int(rng.choice([64, 128])),
        "f16": bool(rng.random() < 0.3),
        "G": 128 * int(rng.integers(0, 5)),
        "prows": int(rng.integers(2, 17)),
        "kb": int(rng.choice([64, 128])),
        "bnhd": bool(rng.random() < 0.4),
        "groups": int(rng.choice([0, 0, 3, 8, 37])),
        "drop": float(rng.choice([0.0, 0.0, 0.5, 1.0])),
        "seed": int(rng.integers(1, 1 << 30)),
    }
    c["N"] = c["G"] + 128 * c["prows"]
    # unpaired 64-query tables, ascending unique blocks: every row with the global prefix first
    # (pair_metadata requires it, paired_metadata.py:26-51), and the same rows with the prefix
    # dropped on some of them (sparse_attention accepts those)
    rows, blocks, prefix = 2 * c["prows"], c["N"] // 64, c["G"] // 64
    width = prefix + 12
    tables = {}
    for name in ("with_prefix", "some_dropped"):
        tables[name] = (np.zeros((rows, width), np.int32), np.zeros(rows, np.int32))
    for r in range(rows):
        size = int(rng.integers(1, min(12, blocks - prefix) + 1))
        extra = np.sort(rng.choice(np.arange(prefix, blocks), size=size, replace=False))
        drop = rng.random() < c["drop"]
        for name, keep in (("with_prefix", True), ("some_dropped", not drop)):
            row = np.concatenate([np.arange(prefix) if keep else [], extra]).astype(np.int32)
            ids, counts = tables[name]
            ids[r, : len(row)] = row
            counts[r] = len(row)
    return c, tables


def _layout(x, bnhd, device):
    x = x.to(device)
    return x.transpose(1, 2).contiguous().transpose(1, 2) if bnhd else x


@pytest.fixture
def groups_setter(monkeypatch):
    from hilberta_amd import paired_kernel, sparse_kernel

    def set_groups(n):
        monkeypatch.setattr(paired_kernel, "NUM_GROUPS", n)
        monkeypatch.setattr(sparse_kernel, "NUM_GROUPS", n)

    return set_groups


@pytest.mark.parametrize("case", range(CASES))
def test_random_tables(hip_device, groups_setter, case):
    from hilberta_amd.paired_kernel import paired_attention
    from hilberta_amd.sparse_kernel import sparse_attention

    c, tables = _draw(case)
    groups_setter(c["groups"])
    B, H, N, D, G = c["B"], c["H"], c["N"], c["D"], c["G"]
    dtype = torch.float16 if c["f16"] else torch.bfloat16
    name = (f"case {case}: B={B} H={H} N={N} D={D} {'fp16' if c['f16'] else 'bf16'} G={G} "
            f"KB{c['kb']} {'BNHD' if c['bnhd'] else 'BHND'} groups={c['groups']} drop={c['drop']}")
    say(name)
    q, k, v = A.seeded_qkv(B, H, N, D, seed=c["seed"], dtype=dtype)
    qd, kd, vd = (_layout(x, c["bnhd"], hip_device) for x in (q, k, v))

    ids, counts = tables["with_prefix"]
    meta = T.pair_metadata(ids, counts, tokens=N, global_tokens=G, key_block_size=c["kb"])
    lse = torch.empty(B, H, N, dtype=torch.float32, device=hip_device)
    out = paired_attention(qd, kd, vd, device_paired(meta, hip_device), lse=lse)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.stride() == qd.stride()
    mask = A.paired_mask(meta["kv_indices"], meta["kv_flags"], meta["kv_counts"], tokens=N,
                         global_tokens=G, key_block_size=c["kb"])
    ref_o, ref_l = A.masked_attention(q, k, v, mask)
    compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"{name} paired_attention")

    ids, counts = tables["some_dropped"]
    lse2 = torch.empty(B, H, N, dtype=torch.float32, device=hip_device)
    out2 = sparse_attention(qd, kd, vd, torch.from_numpy(ids).to(hip_device),
                            torch.from_numpy(counts).to(hip_device), global_tokens=G, lse=lse2)
    torch.cuda.synchronize()
    mask2 = A.explicit_mask(ids, counts, tokens=N, global_tokens=G)
    ref_o2, ref_l2 = A.masked_attention(q, k, v, mask2)
    compare(out2.cpu(), lse2.cpu(), ref_o2, ref_l2, f"{name} sparse_attention")


RAGGED_CASES = 16


def _draw_ragged(case):
    """Shapes the paired layout covers only with an overhanging half: a global prefix of any
    multiple of 64 (0-576) and any number of 64-query rows (1-33, odd or even)."""
    rng = np.random.default_rng(9700 + case)
    c = {
        "B": int(rng.integers(1, 3)),
        "H": int(rng.integers(1, 5)),
        "D": int(rng.choice([64, 128])),
        "f16": bool(rng.random() < 0.3),
        "G": 64 * int(rng.integers(0, 10)),
        "rows": int(rng.integers(1, 34)),
        "bnhd": bool(rng.random() < 0.4),
        "groups": int(rng.choice([0, 0, 3, 8])),
        "drop": float(rng.choice([0.0, 0.5, 1.0])),
        "seed": int(rng.integers(1, 1 << 30)),
    }
    c["N"] = c["G"] + 64 * c["rows"]
    blocks, prefix = c["N"] // 64, c["G"] // 64
    width = prefix + 12
    ids, counts = np.zeros((c["rows"], width), np.int32), np.zeros(c["rows"], np.int32)
    for r in range(c["rows"]):
        size = int(rng.integers(1, min(12, blocks - prefix) + 1))
        extra = np.sort(rng.choice(np.arange(prefix, blocks), size=size, replace=False))
        keep = rng.random() >= c["drop"]
        row = np.concatenate([np.arange(prefix) if keep else [], extra]).astype(np.int32)
        ids[r, : len(row)] = row
        counts[r] = len(row)
    return c, ids, counts


@pytest.mark.parametrize("case", range(RAGGED_CASES))
def test_random_ragged_tables(hip_device, groups_setter, case):
    """sparse_attention on tables whose rows pair only with an overhanging half (odd row counts,
    global prefixes that are odd multiples of 64), against the fp32 explicit-mask oracle."""
    from hilberta_amd.sparse_kernel import sparse_attention

    c, ids, counts = _draw_ragged(case)
    groups_setter(c["groups"])
    B, H, N, D, G = c["B"], c["H"], c["N"], c["D"], c["G"]
    dtype = torch.float16 if c["f16"] else torch.bfloat16
    name = (f"ragged case {case}: B={B} H={H} N={N} D={D} {'fp16' if c['f16'] else 'bf16'} G={G} "
            f"rows={c['rows']} {'BNHD' if c['bnhd'] else 'BHND'} groups={c['groups']} drop={c['drop']}")
    say(name)
    q, k, v = A.seeded_qkv(B, H, N, D, seed=c["seed"], dtype=dtype)
    qd, kd, vd = (_layout(x, c["bnhd"], hip_device) for x in (q, k, v))
    lse = torch.full((B, H, N), float("nan"), dtype=torch.float32, device=hip_device)
    out = sparse_attention(qd, kd, vd, torch.from_numpy(ids).to(hip_device),
                           torch.from_numpy(counts).to(hip_device), global_tokens=G, lse=lse)
    torch.cuda.synchronize()
    ref_o, ref_l = A.masked_attention(q, k, v, A.explicit_mask(ids, counts, tokens=N, global_tokens=G))
    compare(out.cpu(), lse.cpu(), ref_o, ref_l, name)
