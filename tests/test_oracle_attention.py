"""Pins the fp32 attention oracle (oracle/attention.py) on the CPU."""

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import topology as T


def _tiny_tables():
    # 6 blocks of 64 tokens: 2 global, 4 ordinary (the reference's hand example shape)
    ids = np.array([[0, 1, 2, 4], [0, 1, 3, 5], [0, 1, 4, 5], [0, 1, 4, 5]], dtype=np.int32)
    counts = np.array([4, 4, 3, 4], dtype=np.int32)
    return ids, counts


def test_full_tables_equal_library_sdpa():
    q, k, v = A.seeded_qkv(1, 2, 384, 64, dtype=torch.float32)
    nb = 6
    ids = np.tile(np.arange(nb, dtype=np.int32), (4, 1))
    counts = np.full(4, nb, dtype=np.int32)
    mask = A.explicit_mask(ids, counts, tokens=384, global_tokens=128)
    assert mask.all()
    out, lse = A.masked_attention(q, k, v, mask)
    ref = F.scaled_dot_product_attention(q, k, v)
    assert torch.allclose(out, ref, atol=2e-6, rtol=1e-5)
    ref_lse = torch.logsumexp((q @ k.transpose(-1, -2)) / 8.0, -1)
    assert torch.allclose(lse, ref_lse, atol=1e-5)


def test_masked_matches_library_sdpa_with_mask():
    q, k, v = A.seeded_qkv(2, 2, 384, 128, dtype=torch.float32, seed=1)
    ids, counts = _tiny_tables()
    mask = A.explicit_mask(ids, counts, tokens=384, global_tokens=128)
    out, _ = A.masked_attention(q, k, v, mask, scale=0.1)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=0.1)
    assert torch.allclose(out, ref, atol=2e-6, rtol=1e-5)


def test_float64_brute_force_rows():
    q, k, v = A.seeded_qkv(1, 1, 384, 64, dtype=torch.float32, seed=3)
    ids, counts = _tiny_tables()
    mask = A.explicit_mask(ids, counts, tokens=384, global_tokens=128)
    out, lse = A.masked_attention(q, k, v, mask)
    qd, kd, vd = (x[0, 0].double().numpy() for x in (q, k, v))
    m = mask.numpy()
    for row in (0, 127, 128, 191, 200, 255, 300, 383):
        keys = np.nonzero(m[row])[0]
        s = np.array([qd[row] @ kd[j] for j in keys]) / math.sqrt(64)
        top = s.max()
        w = np.exp(s - top)
        expect = (w[:, None] * vd[keys]).sum(0) / w.sum()
        assert np.allclose(out[0, 0, row].numpy(), expect, atol=2e-6)
        assert abs(lse[0, 0, row].item() - (top + math.log(w.sum()))) < 2e-5
    # row 256..319 is query block 2: count 3 -> blocks 0,1,4 only
    assert m[256, :128].all() and m[256, 256:320].all() and not m[256, 128:256].any()


def test_block_formulation_equals_dense_mask():
    ids, counts = _tiny_tables()
    q, k, v = A.seeded_qkv(1, 2, 384, 64, dtype=torch.bfloat16, seed=5)
    mask = A.explicit_mask(ids, counts, tokens=384, global_tokens=128)
    o1, l1 = A.masked_attention(q, k, v, mask)
    o2, l2 = A.block_sparse_attention(q, k, v, ids, counts, global_tokens=128)
    assert torch.allclose(o1, o2, atol=2e-6) and torch.allclose(l1, l2, atol=2e-6)


def test_paired_and_unpaired_masks_agree():
    plan = T.bridge_k_plan(16, 3, False, grid_size=64)
    for phase in plan["phases"]:
        for kb in (64, 128):
            meta = T.pair_metadata(phase["kv_indices"], phase["kv_counts"],
                                   tokens=plan["total_tokens"], global_tokens=plan["global_tokens"],
                                   key_block_size=kb)
            a = A.explicit_mask(phase["kv_indices"], phase["kv_counts"], tokens=plan["total_tokens"],
                                global_tokens=plan["global_tokens"])
            b = A.paired_mask(meta["kv_indices"], meta["kv_flags"], meta["kv_counts"],
                              tokens=plan["total_tokens"], global_tokens=plan["global_tokens"],
                              key_block_size=kb)
            assert torch.equal(a, b)


def test_seeded_inputs_are_device_independent_and_ordered():
    q, k, v = A.seeded_qkv(1, 1, 4, 8, dtype=torch.float32)
    gen = torch.Generator("cpu").manual_seed(2707)
    assert torch.equal(q, torch.randn((1, 1, 4, 8), generator=gen))
    assert torch.equal(k, torch.randn((1, 1, 4, 8), generator=gen))
    assert torch.equal(v, torch.randn((1, 1, 4, 8), generator=gen))
