"""Exact 128-query paired block-sparse attention: the default inference entry point.

Drop-in for the reference module hilberta/paired_kernel.py: ``paired_attention`` keeps its
signature, host-side checks and error messages (paired_kernel.py:97-172) and launches the gfx950
HIP kernel ``hb_paired_fwd`` in place of the Triton ``_paired_fwd``.  Query halves of a paired row
share K/V loads but keep their own masks and softmax denominators (flag bit half + 2*key_half).
"""

from __future__ import annotations

import math
from numbers import Integral, Real

import torch

from .sparse_kernel import (
    LOG2E,
    _check_lse,
    _check_vector_layout,
    _non_overlapping_strides,
    _tensor_byte_span,
)


# Persistent workgroup count for hb_paired_fwd; 0 lets the library choose (2 per compute unit; 3
# for D = 64 calls with at least two items per workgroup).
NUM_GROUPS = 0


def _paired_fwd(q, k, v, out, lse, metadata, scale_log2, all_queries):
    """Launch through the operator hilberta_hip::paired_fwd on the current stream (module-level so
    tests can patch it)."""
    from . import ops

    ops.paired_fwd(q, k, v, out, lse, metadata.kv_indices, metadata.kv_flags, metadata.kv_counts,
                   int(metadata.global_tokens), int(metadata.key_block_size), float(scale_log2),
                   bool(all_queries), int(NUM_GROUPS))


def paired_attention(
    q, k, v, metadata, *, global_strategy="flash", num_warps=4, num_stages=2, scale=None, out=None,
    lse=None,
):
    """Exact inference attention over paired tables; metadata validated on CPU before transfer.

    Input checks inspect host-side tensor properties only: no device values are read, nothing
    synchronises, no mask is built and Q/K/V are not packed.  Both ``global_strategy`` values run
    the single HIP kernel (global query rows attend every key block in the same launch); the
    tuning keywords are validated as in the reference but select no code path.  ``lse`` may be a
    contiguous float32 [B,H,N] tensor that receives the natural-log row logsumexp.
    """
    if q.ndim != 4 or k.shape != q.shape or v.shape != q.shape or any(x <= 0 for x in q.shape):
        raise ValueError("Equal nonempty B,H,N,D Q/K/V required")
    if q.shape[-1] not in (64, 128) or any(x.stride(-1) != 1 for x in (q, k, v)):
        raise ValueError("D64 or128 must be contiguous")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("Q/K/V must share BF16/FP16 dtype")
    if not q.is_cuda or k.device != q.device or v.device != q.device:
        raise ValueError("Q/K/V must be on the same CUDA device")
    if any(any(s <= 0 for s in x.stride()[:3]) for x in (q, k, v)):
        raise ValueError("Positive Q/K/V outer strides required")
    if torch.is_grad_enabled() and any(x.requires_grad for x in (q, k, v)):
        raise ValueError("Inference only; disable autograd")
    for name in ("tokens", "global_tokens", "key_block_size"):
        value = getattr(metadata, name)
        if isinstance(value, bool) or not isinstance(value, Integral):
            raise TypeError("Integer metadata shape fields required")
    N, G = metadata.tokens, metadata.global_tokens
    if q.shape[-2] != N or G % 128 or N % 128 or not 0 <= G < N or metadata.key_block_size not in (64, 128):
        raise ValueError("Metadata/token shape mismatch or invalid128-token alignment")
    rows = (N - G) // 128
    if metadata.kv_indices.ndim != 2 or metadata.kv_indices.shape[0] != rows or metadata.kv_indices.shape[1] < 1:
        raise ValueError("Paired index shape must match ordinary query pairs")
    if metadata.kv_flags.shape != metadata.kv_indices.shape or metadata.kv_counts.shape != (rows,):
        raise ValueError("Paired flag/count shape mismatch")
    for x in (metadata.kv_indices, metadata.kv_flags, metadata.kv_counts):
        if x.device != q.device or x.dtype != torch.int32 or not x.is_contiguous():
            raise ValueError("Cached CUDA contiguous int32 metadata required")
    if global_strategy not in ("flash", "triton"):
        raise ValueError("Invalid global strategy")
    if any(isinstance(x, bool) or not isinstance(x, Integral) for x in (num_warps, num_stages)):
        raise TypeError("Integer launch tuning required")
    if num_warps not in (4, 8) or num_stages not in (1, 2, 3, 4):
        raise ValueError("Invalid launch tuning")
    if scale is not None and (isinstance(scale, bool) or not isinstance(scale, Real)):
        raise TypeError("scale must be a real scalar, never a tensor")
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("Positive finite scale required")
    if out is not None:
        if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(-1) != 1:
            raise ValueError("Output must match Q shape/dtype/device with contiguous D")
        if any(s <= 0 for s in out.stride()) or not _non_overlapping_strides(out):
            raise ValueError("Positive non-overlapping output strides required")
        if torch.is_grad_enabled() and out.requires_grad:
            raise ValueError("Inference output cannot require gradients")
        begin, end = _tensor_byte_span(out)
        for x in (q, k, v, metadata.kv_indices, metadata.kv_flags, metadata.kv_counts):
            first, last = _tensor_byte_span(x)
            if begin < last and first < end:
                raise ValueError("Output cannot alias inputs or metadata")
    else:
        out = torch.empty_like(q)
    _check_lse(lse, q)
    _check_vector_layout((q, k, v, out))
    _paired_fwd(q, k, v, out, lse, metadata, scale * LOG2E, True)
    return out
