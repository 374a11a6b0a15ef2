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


def index_select_rows(x, dim, index, *, out=None, error=None, check=False):
    """Gather rows of ``x`` along ``dim`` by ``index`` (int64, on x's device) with the HIP kernel.

    Indices are trusted by default: the persistent-layout orders come from the plan builder,
    which checks them once (every order it returns is a permutation of the image tokens), and the
    per-forward gather must not synchronise.  An out-of-range index is then skipped (its row of
    the output is left unwritten; nothing outside ``x`` or the output is touched).  ``check=True``
    raises IndexError as ``index_select`` does (reference flux_adapter.py:209-212), at the cost of
    one host synchronisation.  ``error`` may instead be a device int32 scalar tensor that the
    kernel sets to 1 on an out-of-range index, for callers that check it later.  Without ``out``,
    ``error`` and ``check`` this is the operator ``torch.ops.hilberta_hip.gather_rows``.
    """
    _lib.require_gpu(x, index)
    dim = dim % x.ndim
    if index.dtype != torch.int64 or index.ndim != 1 or index.device != x.device:
        raise ValueError("index must be a 1-D int64 tensor on x's device")
    if check:
        err = torch.zeros(1, dtype=torch.int32, device=x.device) if error is None else error
        res = gather_into(x, dim, index, out=out, error=err)
        if int(err.item()):
            raise IndexError("index out of range in self")
        return res
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
