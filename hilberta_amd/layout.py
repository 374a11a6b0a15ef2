"""Hilbert permutation of token rows on the GPU (HIP gather, csrc/layout.hip).

Replaces the reference's ``x.index_select(dim, order)`` at transformer entry/exit
(hilberta/flux_adapter.py:209-212, :243) and at sampling entry/exit
(hilberta/sampling_layout.py:96-97, :110): ``index_select_rows(x, dim, index)`` returns
``x.index_select(dim, index)`` bit for bit.  The slice x[..., i, ...] along ``dim`` must be
contiguous (true for [B, n, C] latents, [n, 3] ids and [B, N, H, D] projections); outer
dimensions may have any stride that keeps them uniformly spaced.
"""

from __future__ import annotations

import math

import torch

from . import _lib


def _outer_stride(x, dim):
    """Single stride walking every index of the dims before ``dim``, or None if none exists."""
    shape, stride = x.shape[:dim], x.stride()[:dim]
    outer = math.prod(shape)
    if outer <= 1:
        return outer, 0
    dims = [(s, st) for s, st in zip(shape, stride) if s > 1]
    for (s0, st0), (s1, st1) in zip(dims[1:], dims[:-1]):
        if st1 != st0 * s0:
            return outer, None
    return outer, dims[-1][1]


def index_select_rows(x, dim, index, *, out=None, error=None):
    """Gather rows of ``x`` along ``dim`` by ``index`` (int64, on x's device) with the HIP kernel.

    ``error`` may be a device int32 scalar tensor that is set to 1 if an index was out of range
    (such rows are left unwritten); without it, indices are trusted (validated at plan setup).
    Without ``out`` and ``error`` this is the operator ``torch.ops.hilberta_hip.gather_rows``.
    """
    _lib.require_gpu(x, index)
    dim = dim % x.ndim
    if index.dtype != torch.int64 or index.ndim != 1 or index.device != x.device:
        raise ValueError("index must be a 1-D int64 tensor on x's device")
    if out is None and error is None:
        from . import ops

        return ops.gather_rows(x, dim, index)
    return gather_into(x, dim, index, out=out, error=error)


def gather_into(x, dim, index, *, out=None, error=None):
    """The hb_gather_rows launch behind index_select_rows (arguments already checked there)."""
    inner = x.shape[dim + 1 :]
    row_elems = math.prod(inner)
    expect = 1
    for s, st in zip(reversed(inner), reversed(x.stride()[dim + 1 :])):
        if s > 1 and st != expect:
            raise ValueError("index_select_rows needs the dims after `dim` to be contiguous")
        expect *= s
    outer, src_outer = _outer_stride(x, dim)
    if src_outer is None:
        x = x.contiguous()
        outer, src_outer = _outer_stride(x, dim)
    shape = list(x.shape)
    shape[dim] = index.numel()
    if out is None:
        out = torch.empty(shape, dtype=x.dtype, device=x.device)
    elif list(out.shape) != shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("out must be contiguous with the gathered shape and x's dtype")
    es = x.element_size()
    dst_outer = index.numel() * row_elems
    lib = _lib.load()
    rc = lib.hb_gather_rows(
        x.data_ptr(), out.data_ptr(), index.data_ptr(), index.numel(), outer, src_outer * es,
        dst_outer * es, x.stride(dim) * es, row_elems * es, row_elems * es, x.shape[dim],
        error.data_ptr() if error is not None else None, _lib.stream_ptr(x.device),
    )
    _lib.check(rc, "hb_gather_rows")
    return out


def permute_tokens(x, order, dim=1):
    """Raster -> persistent Hilbert layout: x.index_select(dim, order)."""
    return index_select_rows(x, dim, order)


def unpermute_tokens(x, inverse_order, dim=1):
    """Persistent layout -> raster: x.index_select(dim, inverse_order)."""
    return index_select_rows(x, dim, inverse_order)
