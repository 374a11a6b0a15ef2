"""Tables whose rows may start with an entry that only one query half sees.

paired_attention admits a zero-token global prefix (reference paired_kernel.py:127: 0 <= G < N)
and sparse_attention admits tables without the global prefix (its launch checks never ask for
one, sparse_kernel.py:188-250), which it pairs on the device and runs on the paired kernel.  The
reference applies every entry's own flags, entry 0 included (paired_kernel.py:70-84).  With few
persistent workgroups every workgroup runs many items in a row, so each item's first step goes
through the item-to-item hand-over rather than the kernel's start.

Reference: fp32 dense masked attention (oracle/attention.py) with the paired-flag mask or the
unpaired explicit mask, on the CPU.
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import topology as T
from tests.helpers import compare, device_paired, say

pytestmark = pytest.mark.gpu

D = 128


def _random_rows(rows, total_blocks, rng, *, prefix_blocks=0, drop_prefix=0.0, lo=2, hi=9):
    """Unpaired tables: each row lists 1-8 random blocks (ascending, unique); the global prefix
    is listed first unless the row drops it (probability drop_prefix)."""
    width = prefix_blocks + hi
    ids = np.zeros((rows, width), np.int32)
    counts = np.zeros(rows, np.int32)
    for r in range(rows):
        pool = np.arange(prefix_blocks, total_blocks)
        extra = np.sort(rng.choice(pool, size=int(rng.integers(lo, hi)), replace=False))
        keep_prefix = prefix_blocks and rng.random() >= drop_prefix
        row = np.concatenate([np.arange(prefix_blocks) if keep_prefix else [], extra]).astype(np.int32)
        ids[r, : len(row)] = row
        counts[r] = len(row)
    return ids, counts


@pytest.fixture
def few_groups(monkeypatch):
    from hilberta_amd import paired_kernel, sparse_kernel

    def set_groups(n):
        monkeypatch.setattr(paired_kernel, "NUM_GROUPS", n)
        monkeypatch.setattr(sparse_kernel, "NUM_GROUPS", n)

    return set_groups


@pytest.mark.parametrize("key_block_size", [64, 128])
@pytest.mark.parametrize("groups", [8, 3, 1, 0])
def test_paired_zero_global_prefix(hip_device, few_groups, key_block_size, groups):
    """G = 0: every paired row's first union entry has its own flags (1, 2 or 3)."""
    from hilberta_amd.paired_kernel import paired_attention

    few_groups(groups)
    rows, heads = 40, 4
    N = 64 * rows
    rng = np.random.default_rng(31 + key_block_size)
    ids, counts = _random_rows(rows, N // 64, rng)
    meta_np = T.pair_metadata(ids, counts, tokens=N, global_tokens=0, key_block_size=key_block_size)
    first = meta_np["kv_flags"][:, 0]
    if key_block_size == 64:
        assert ((first == 1) | (first == 2)).sum() >= 4, "needs rows whose first entry one half sees"
    else:
        assert ((first & 3) == 0).sum() >= 2, "needs rows whose first 64-key half nobody sees"
        assert (((first & 3) == 1) | ((first & 3) == 2)).sum() >= 2
    q, k, v = A.seeded_qkv(1, heads, N, D, seed=17)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    say(f"case paired G=0 KB{key_block_size} groups={groups} N={N}")
    lse = torch.empty(1, heads, N, dtype=torch.float32, device=hip_device)
    out = paired_attention(qd, kd, vd, device_paired(meta_np, hip_device), lse=lse)
    torch.cuda.synchronize()
    mask = A.paired_mask(meta_np["kv_indices"], meta_np["kv_flags"], meta_np["kv_counts"], tokens=N,
                         global_tokens=0, key_block_size=key_block_size)
    ref_o, ref_l = A.masked_attention(q, k, v, mask)
    compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"paired G=0 KB{key_block_size} groups={groups}")


@pytest.mark.parametrize("global_tokens", [512, 0])
@pytest.mark.parametrize("groups", [8, 0])
def test_sparse_attention_prefixless_tables(hip_device, few_groups, global_tokens, groups):
    """Unpaired tables without the global prefix (some rows keep it, most drop it) go through the
    device pairing and the paired kernel; global query rows still attend every key."""
    from hilberta_amd.sparse_kernel import sparse_attention

    few_groups(groups)
    rows, heads = 48, 3
    G = global_tokens
    N = G + 64 * rows
    rng = np.random.default_rng(7 + G)
    ids, counts = _random_rows(rows, N // 64, rng, prefix_blocks=G // 64, drop_prefix=0.7, lo=1)
    q, k, v = A.seeded_qkv(1, heads, N, D, seed=19)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    say(f"case sparse_attention prefix-less G={G} groups={groups} N={N}")
    lse = torch.empty(1, heads, N, dtype=torch.float32, device=hip_device)
    out = sparse_attention(qd, kd, vd, torch.from_numpy(ids).to(hip_device),
                           torch.from_numpy(counts).to(hip_device), global_tokens=G, lse=lse)
    torch.cuda.synchronize()
    mask = A.explicit_mask(ids, counts, tokens=N, global_tokens=G)
    ref_o, ref_l = A.masked_attention(q, k, v, mask)
    compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"sparse prefix-less G={G} groups={groups}")
