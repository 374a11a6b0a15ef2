"""Exact block-sparse FLUX self-attention on a persistent token layout (unpaired tables).

Drop-in for the reference module hilberta/sparse_kernel.py: the same call surface
(``sparse_attention``, ``validate_metadata``, ``explicit_mask``, ``_check_inputs``,
``_tensor_byte_span``, ``_non_overlapping_strides``) with the same host-side checks and error
messages, launching the gfx950 HIP kernels (operator hilberta_hip::sparse_fwd) instead of the
Triton ``_block_sparse_fwd``.

Q/K/V are [batch, heads, tokens, head_dim] views; physical token order is a fully connected
global prefix followed by ordinary 64-token query blocks, each listing its allowed key blocks.
Inference only; launches are asynchronous on the current stream with no host synchronisation.
``explicit_mask`` builds the dense mask of a table for correctness checks; no kernel uses it.
"""

from __future__ import annotations

import math
from numbers import Integral, Real

import torch


LOG2E = 1.4426950408889634

# Persistent workgroup count for the attention launches of sparse_attention; 0 lets the library
# choose (2 per compute unit; 3 for paired D = 64 calls with at least two items per workgroup,
# which covers pairable tables, since sparse_attention runs those on the paired kernel).
NUM_GROUPS = 0


def validate_metadata(
    kv_indices, kv_counts, *, tokens, global_tokens=768, block_size=64, require_global_prefix=True
):
    """Run once on CPU metadata before launch; never called in the hot path.

    Same checks, messages and returned entry counts as reference sparse_kernel.py:100-152.
    Duplicate K/V blocks are rejected (processing one twice would change the denominator);
    padded entries beyond each count are ignored.
    """
    if block_size != 64:
        raise ValueError("This kernel currently requires 64-token physical blocks")
    if any(isinstance(v, bool) or not isinstance(v, Integral) for v in (tokens, global_tokens)):
        raise TypeError("tokens and global_tokens must be integers")
    if not (0 <= global_tokens < tokens) or tokens % block_size or global_tokens % block_size:
        raise ValueError("tokens/global prefix must be block-aligned with at least one ordinary block")
    if kv_indices.dtype != torch.int32 or kv_counts.dtype != torch.int32:
        raise TypeError("Block metadata must use int32")
    if kv_indices.device.type != "cpu" or kv_counts.device.type != "cpu":
        raise ValueError("Validate CPU metadata before transferring/caching it on GPU")
    rows = (tokens - global_tokens) // block_size
    if kv_indices.ndim != 2 or kv_indices.shape[0] != rows or kv_indices.shape[1] < 1:
        raise ValueError("kv_indices must be [ordinary_query_blocks, max_KV_blocks]")
    if kv_counts.shape != (rows,):
        raise ValueError("kv_counts must have one entry per ordinary query block")
    if not kv_indices.is_contiguous() or not kv_counts.is_contiguous():
        raise ValueError("Metadata must be contiguous")
    nblocks, global_blocks = tokens // block_size, global_tokens // block_size
    counts = kv_counts.tolist()
    width = kv_indices.shape[1]
    bad = [r for r, c in enumerate(counts) if not 1 <= c <= width]
    if bad:
        raise ValueError(f"Invalid K/V count in ordinary query block {bad[0]}")
    # vectorised equivalent of the per-row loop: range, uniqueness and global prefix
    col = torch.arange(width)[None, :]
    active = col < kv_counts[:, None].long()
    ids = kv_indices.long()
    out_of_range = active & ((ids < 0) | (ids >= nblocks))
    keyed = torch.where(active, ids, -1 - col)  # padding can never collide with a real id
    dup = (keyed.sort(1).values.diff(dim=1) == 0).any(1)
    bad_rows = (out_of_range.any(1) | dup).nonzero()
    if len(bad_rows):
        raise ValueError(f"Out-of-range or duplicate K/V blocks in row {int(bad_rows[0])}")
    if require_global_prefix and global_blocks:
        present = ((ids[:, :, None] == torch.arange(global_blocks)) & active[:, :, None]).any(1)
        missing = (~present.all(1)).nonzero()
        if len(missing):
            raise ValueError(f"Row {int(missing[0])} misses global-prefix keys")
    ordinary_entries = sum(counts) * block_size * block_size
    return {
        "tokens": tokens,
        "global_tokens": global_tokens,
        "block_size": block_size,
        "ordinary_query_blocks": rows,
        "min_kv_blocks": min(counts),
        "max_kv_blocks": max(counts),
        "global_directed_entries": global_tokens * tokens,
        "ordinary_directed_entries": ordinary_entries,
        "total_directed_entries": global_tokens * tokens + ordinary_entries,
    }


def explicit_mask(kv_indices, kv_counts, *, tokens, global_tokens=768, block_size=64):
    """Dense [tokens, tokens] boolean mask of unpaired CPU tables, for correctness checks only
    (reference sparse_kernel.py:155-166; the kernels never build it).  The tables are validated
    first; global query rows see every key, ordinary query block r the key blocks it lists."""
    validate_metadata(kv_indices, kv_counts, tokens=tokens, global_tokens=global_tokens,
                      block_size=block_size)
    key_blocks, global_blocks = tokens // block_size, global_tokens // block_size
    listed = torch.arange(kv_indices.shape[1])[None, :] < kv_counts[:, None].long()
    row = torch.arange(kv_indices.shape[0])[:, None].expand(kv_indices.shape)
    blocks = torch.zeros(key_blocks, key_blocks, dtype=torch.bool)
    blocks[:global_blocks] = True
    blocks[global_blocks + row[listed], kv_indices.long()[listed]] = True
    return blocks.repeat_interleave(block_size, 0).repeat_interleave(block_size, 1)


def _tensor_byte_span(tensor):
    """Conservative [begin, end) byte interval of a strided view (host metadata only)."""
    begin = tensor.data_ptr()
    extent = 1 + sum((size - 1) * stride for size, stride in zip(tensor.shape, tensor.stride()))
    return begin, begin + extent * tensor.element_size()


def _non_overlapping_strides(tensor):
    extent = 1
    for stride, size in sorted(
        (stride, size) for stride, size in zip(tensor.stride(), tensor.shape) if size > 1
    ):
        if stride < extent:
            return False
        extent += (size - 1) * stride
    return True


def _check_inputs(q, k, v, kv_indices, kv_counts, global_tokens, block_size, out):
    """Host-side launch checks of reference sparse_kernel.py:188-250 (same messages)."""
    if q.ndim != 4 or k.shape != q.shape or v.shape != q.shape or any(s <= 0 for s in q.shape):
        raise ValueError("Q/K/V must have equal, nonempty [B,H,N,D] shapes")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("Q/K/V must share FP16 or BF16 dtype")
    if not q.is_cuda or k.device != q.device or v.device != q.device:
        raise ValueError("Q/K/V must be on one CUDA device")
    if torch.is_grad_enabled() and any(x.requires_grad for x in (q, k, v)):
        raise ValueError("sparse_attention is inference-only; disable autograd before calling")
    if q.shape[-1] not in (64, 128) or any(x.stride(-1) != 1 for x in (q, k, v)):
        raise ValueError("D must be64 or128 and contiguous; outer strides may differ")
    if any(any(stride <= 0 for stride in x.stride()[:3]) for x in (q, k, v)):
        raise ValueError("Q/K/V outer strides must be positive")
    if any(isinstance(v_, bool) or not isinstance(v_, Integral) for v_ in (global_tokens, block_size)):
        raise TypeError("global_tokens and block_size must be integers")
    n = q.shape[-2]
    if block_size != 64 or n % block_size or global_tokens % block_size or not 0 <= global_tokens < n:
        raise ValueError("N and global_tokens must align to64, with ordinary queries remaining")
    rows = (n - global_tokens) // block_size
    if (
        kv_indices.ndim != 2
        or kv_indices.shape[0] != rows
        or kv_indices.shape[1] < 1
        or kv_counts.shape != (rows,)
    ):
        raise ValueError("Metadata shape does not match the ordinary query partition")
    if any(
        x.device != q.device or x.dtype != torch.int32 or not x.is_contiguous()
        for x in (kv_indices, kv_counts)
    ):
        raise ValueError("Metadata must be cached contiguous CUDA int32 tensors on the Q device")
    if out is not None:
        if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(-1) != 1:
            raise ValueError(
                "Provided output must match Q shape/dtype/device with contiguous last dimension"
            )
        if any(stride <= 0 for stride in out.stride()) or not _non_overlapping_strides(out):
            raise ValueError("Provided output must have positive, non-overlapping strides")
        if torch.is_grad_enabled() and out.requires_grad:
            raise ValueError("An inference output cannot require gradients")
        out_lo, out_hi = _tensor_byte_span(out)
        for tensor in (q, k, v, kv_indices, kv_counts):
            in_lo, in_hi = _tensor_byte_span(tensor)
            if out_lo < in_hi and in_lo < out_hi:
                raise ValueError("Provided output must not alias Q/K/V or metadata storage")


def _check_vector_layout(tensors):
    """The HIP kernel moves 16-byte vectors: base pointers 16-byte aligned, strides multiple of 8."""
    for x in tensors:
        if x.data_ptr() % 16 or any(s % 8 for s in x.stride()[:3]):
            raise ValueError(
                "HIP attention needs 16-byte aligned Q/K/V/out with outer strides a multiple of 8"
            )


def _check_lse(lse, q):
    if lse is None:
        return
    B, H, N, _ = q.shape
    if (
        not isinstance(lse, torch.Tensor)
        or lse.shape != (B, H, N)
        or lse.dtype != torch.float32
        or lse.device != q.device
        or not lse.is_contiguous()
    ):
        raise ValueError("lse must be a contiguous float32 [B,H,N] tensor on the Q device")


def _strides(q, k, v, out):
    return [s for x in (q, k, v, out) for s in x.stride()[:3]]


def _block_sparse_fwd(q, k, v, out, lse, kv_indices, kv_counts, global_tokens, scale_log2,
                      all_queries):
    """Launch through the operator hilberta_hip::sparse_fwd on the current stream (module-level
    so tests can patch it).  The rows are paired on the device (an odd row count from the end)
    and run on the paired kernel up to 16384 key blocks; see hilberta_amd.ops.sparse_fwd."""
    from . import ops

    ops.sparse_fwd(q, k, v, out, lse, kv_indices, kv_counts, int(global_tokens), float(scale_log2),
                   bool(all_queries), int(NUM_GROUPS))


def sparse_attention(
    q,
    k,
    v,
    kv_indices,
    kv_counts,
    global_tokens=768,
    block_size=64,
    *,
    global_strategy="flash",
    query_block_size=64,
    num_warps=4,
    num_stages=2,
    scale=None,
    out=None,
    lse=None,
):
    """Return the exact mask's attention in the original Q shape/dtype (reference :253-340).

    Both global strategies run the single HIP kernel (global query rows attend every key block in
    the same launch); the tuning keywords are validated as in the reference but select no code
    path.  ``lse`` optionally receives the fp32 [B,H,N] natural-log row logsumexp.  Output
    allocation preserves Q's storage order (e.g. BNHD viewed as BHND).
    """
    _check_inputs(q, k, v, kv_indices, kv_counts, global_tokens, block_size, out)
    if global_strategy not in ("flash", "triton"):
        raise ValueError("global_strategy must be flash or triton")
    if any(
        isinstance(value, bool) or not isinstance(value, Integral)
        for value in (query_block_size, num_warps, num_stages)
    ):
        raise TypeError("Kernel tuning arguments must be integers")
    if query_block_size not in (32, 64) or num_warps not in (4, 8) or num_stages not in (1, 2, 3, 4):
        raise ValueError("Supported tuning: query_block_size32/64, warps4/8, stages1..4")
    if scale is not None and (isinstance(scale, bool) or not isinstance(scale, Real)):
        raise TypeError("scale must be a real Python/NumPy scalar, never a tensor")
    global_tokens = int(global_tokens)
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("Softmax scale must be positive and finite")
    _check_lse(lse, q)
    if out is None:
        out = torch.empty_like(q)
    _check_vector_layout((q, k, v, out))
    _block_sparse_fwd(q, k, v, out, lse, kv_indices, kv_counts, global_tokens, scale * LOG2E, True)
    return out
