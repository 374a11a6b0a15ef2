"""fp32 dense masked attention with per-row logsumexp -- TEST ORACLE ONLY.

Mask semantics follow the reference:
  * ordinary tables: sparse_kernel.explicit_mask (hilberta/sparse_kernel.py:155-166) --
    global query rows see every key, ordinary query block r sees the listed
    64-token key blocks;
  * paired tables: the flag test of the paired kernel
    (hilberta/paired_kernel.py:65, :83-84) -- query half h of paired row r sees
    key half kh of block b iff (flags >> (h + 2*kh)) & 1;
  * text rows and columns are all True (tests/mask_reference.py:71-81).

Softmax and LSE are the textbook definitions in fp32:
  out = softmax(scale * Q K^T masked) V,  lse = logsumexp(scale * Q K^T masked).

Pinned by (tests/test_oracle_attention.py): with all-connection tables the
result equals torch's own scaled_dot_product_attention and torch.logsumexp
(library routines); a float64 per-row loop on tiny inputs; the block-wise
formulation here equals the dense-mask formulation; paired and unpaired masks
of pair_metadata tables are identical.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def explicit_mask(kv_indices, kv_counts, *, tokens, global_tokens, block_size=64):
    """Dense [tokens, tokens] bool mask of unpaired tables (sparse_kernel.py:155-166)."""
    ids = np.asarray(kv_indices)
    counts = np.asarray(kv_counts)
    nb = tokens // block_size
    g = global_tokens // block_size
    blocks = np.zeros((nb, nb), dtype=bool)
    blocks[:g] = True
    for row, count in enumerate(counts.tolist()):
        blocks[g + row, ids[row, :count]] = True
    return torch.from_numpy(blocks.repeat(block_size, 0).repeat(block_size, 1))


def paired_mask(kv_indices, kv_flags, kv_counts, *, tokens, global_tokens, key_block_size=64):
    """Dense [tokens, tokens] bool mask of paired tables (paired_kernel.py:65,79,83-84)."""
    ids = np.asarray(kv_indices)
    flags = np.asarray(kv_flags)
    counts = np.asarray(kv_counts)
    nb = tokens // 64
    g = global_tokens // 64
    ratio = key_block_size // 64
    blocks = np.zeros((nb, nb), dtype=bool)
    blocks[:g] = True
    for row, count in enumerate(counts.tolist()):
        for block, flag in zip(ids[row, :count].tolist(), flags[row, :count].tolist()):
            for half in range(2):
                for kh in range(ratio):
                    if (flag >> (half + 2 * kh)) & 1:
                        blocks[g + 2 * row + half, block * ratio + kh] = True
    return torch.from_numpy(blocks.repeat(64, 0).repeat(64, 1))


def masked_attention(q, k, v, mask, scale=None):
    """fp32 masked attention per (batch, head); returns (out fp32 [B,H,N,D], lse fp32 [B,H,N]).

    ``mask`` is bool [N, N] (True = visible) on the same device as q.  Computed
    one head at a time so the [N, N] score scratch stays one head large.
    """
    B, H, N, D = q.shape
    scale = D ** -0.5 if scale is None else float(scale)
    out = torch.empty((B, H, N, D), dtype=torch.float32, device=q.device)
    lse = torch.empty((B, H, N), dtype=torch.float32, device=q.device)
    neg = torch.tensor(-math.inf, dtype=torch.float32, device=q.device)
    for b in range(B):
        for h in range(H):
            qh = q[b, h].float()
            kh = k[b, h].float().contiguous()
            vh = v[b, h].float()
            s = torch.matmul(qh, kh.t().contiguous()) * scale
            s = torch.where(mask, s, neg)
            row_lse = torch.logsumexp(s, dim=-1)
            p = torch.exp(s - row_lse[:, None])
            out[b, h] = torch.matmul(p, vh)
            lse[b, h] = row_lse
            del s, p
    return out, lse


def block_sparse_attention(q, k, v, kv_indices, kv_counts, *, global_tokens, scale=None,
                           block_size=64, heads=None):
    """Same maths without an [N, N] mask: each ordinary query block attends only its listed blocks.

    Global query rows attend every key.  ``heads`` optionally restricts the
    computation to a subset of head indices (others are left as NaN).
    Returns (out fp32 [B,H,N,D], lse fp32 [B,H,N]).
    """
    B, H, N, D = q.shape
    scale = D ** -0.5 if scale is None else float(scale)
    ids = torch.as_tensor(np.asarray(kv_indices)).long()
    counts = np.asarray(kv_counts).tolist()
    out = torch.full((B, H, N, D), math.nan, dtype=torch.float32, device=q.device)
    lse = torch.full((B, H, N), math.nan, dtype=torch.float32, device=q.device)
    heads = range(H) if heads is None else heads
    G = global_tokens
    for b in range(B):
        for h in heads:
            qh, kh, vh = q[b, h].float(), k[b, h].float(), v[b, h].float()
            if G:
                s = torch.matmul(qh[:G], kh.t().contiguous()) * scale
                row_lse = torch.logsumexp(s, -1)
                out[b, h, :G] = torch.matmul(torch.exp(s - row_lse[:, None]), vh)
                lse[b, h, :G] = row_lse
            for row, count in enumerate(counts):
                q0 = G + row * block_size
                blocks = ids[row, :count]
                cols = (blocks[:, None] * block_size + torch.arange(block_size)).reshape(-1)
                cols = cols.to(q.device)
                s = torch.matmul(qh[q0 : q0 + block_size], kh[cols].t().contiguous()) * scale
                row_lse = torch.logsumexp(s, -1)
                out[b, h, q0 : q0 + block_size] = torch.matmul(torch.exp(s - row_lse[:, None]), vh[cols])
                lse[b, h, q0 : q0 + block_size] = row_lse
    return out, lse


def seeded_qkv(batch, heads, tokens, head_dim, *, seed=2707, dtype=torch.bfloat16):
    """Q, K, V drawn in q, k, v order as fp32 randn from a CPU generator, then cast.

    Device-independent version of the reference harness inputs (benchmark.py:24,28).
    """
    gen = torch.Generator("cpu").manual_seed(seed)
    shape = (batch, heads, tokens, head_dim)
    return [torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype) for _ in range(3)]
