"""torch custom ops over the C ABI (namespace ``hilberta_hip``).

The reference launches its kernels as framework-visible Triton launches (paired_kernel.py:181-204,
sparse_kernel.py:315-339) and gathers with ``index_select`` (flux_adapter.py:209-212, :243).
Here each HIP entry point of include/hilberta_hip.h is a registered operator with a schema, a
fake (shape-only) implementation for tracing, and a real implementation for HIP devices (and,
for pair_rows alone, for the CPU):

  hilberta_hip::paired_fwd(q, k, v, out!, lse!?, kv_indices, kv_flags, kv_counts, global_tokens,
                           key_block_size, scale_log2, all_queries, num_groups) -> ()
  hilberta_hip::sparse_fwd(q, k, v, out!, lse!?, kv_indices, kv_counts, global_tokens,
                           scale_log2, all_queries, num_groups) -> ()
  hilberta_hip::gather_rows(x, dim, index) -> Tensor
  hilberta_hip::pair_rows(kv_indices, kv_counts, total_blocks, key_block_size, paired_width)
                           -> (ids, flags, counts)

The attention ops write into caller-provided outputs (declared mutated), as the reference's
launches write into ``out``.  Argument checks with the reference's messages stay in the Python
entry points (paired_attention, sparse_attention) and run before the op; the library repeats the
cheap ones and reports them as ValueError.  The attention and gather ops have no CPU kernel: on
CPU tensors they raise.  pair_rows is plan setup and also runs on CPU tensors, through the
library's host table builder (hb_pair_rows_host, bit-identical to the device kernel).
"""

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from ._workspace import attention_workspace

_NS = "hilberta_hip"
# key blocks per row hb_pair_rows pairs (include/hilberta_hip.h)
PAIR_MAX_BLOCKS = 16384


def _strides(q, k, v, out):
    return (ctypes.c_int64 * 12)(*[s for x in (q, k, v, out) for s in x.stride()[:3]])


def _dtype_code(q):
    return 1 if q.dtype == torch.float16 else 0


@torch.library.custom_op(f"{_NS}::paired_fwd", mutates_args=("out", "lse"), device_types="cuda")
def paired_fwd(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Optional[Tensor],
               kv_indices: Tensor, kv_flags: Tensor, kv_counts: Tensor, global_tokens: int,
               key_block_size: int, scale_log2: float, all_queries: bool, num_groups: int) -> None:
    """hb_paired_fwd on the current stream (replaces the _paired_fwd launch,
    paired_kernel.py:181-204)."""
    lib = _lib.load()
    B, H, N, D = q.shape
    width = kv_indices.shape[1]
    ws = attention_workspace(q.device, B, H, N, D, global_tokens, width, key_block_size, paired=1,
                             all_queries=all_queries)
    rc = lib.hb_paired_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        lse.data_ptr() if lse is not None else None, _strides(q, k, v, out), B, H, N, D,
        _dtype_code(q), kv_indices.data_ptr(), kv_flags.data_ptr(), kv_counts.data_ptr(), width,
        global_tokens, key_block_size, int(all_queries), scale_log2, ws.data_ptr(), ws.numel(),
        num_groups, _lib.stream_ptr(q.device))
    _lib.check(rc, "hb_paired_fwd")


@paired_fwd.register_fake
def _(q, k, v, out, lse, kv_indices, kv_flags, kv_counts, global_tokens, key_block_size,
      scale_log2, all_queries, num_groups):
    return None


@torch.library.custom_op(f"{_NS}::sparse_fwd", mutates_args=("out", "lse"), device_types="cuda")
def sparse_fwd(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Optional[Tensor],
               kv_indices: Tensor, kv_counts: Tensor, global_tokens: int, scale_log2: float,
               all_queries: bool, num_groups: int) -> None:
    """Unpaired 64-query tables (replaces the _block_sparse_fwd launch, sparse_kernel.py:315-339).

    With at most PAIR_MAX_BLOCKS key blocks, rows 2r, 2r + 1 are merged on the device by hb_pair_rows, as
    pair_metadata does (paired_metadata.py:26-51), and run on hb_paired_fwd: a 128-query item
    keeps two waves per SIMD busy where a 64-query item keeps one (1.7-1.85x faster).  An odd row
    count is paired from the end, its first paired row carrying an empty half that reaches into
    the global prefix and is never stored; a global prefix that is an odd multiple of 64 leaves a
    last global tile whose upper half is never stored either.  Every query sees the same key
    blocks in the same ascending order with the same arithmetic; the other half's blocks are
    masked to exact zeros.  The paired tables are padded to min(2 * width, N / 64) entries, which
    needs no host synchronisation.  Longer sequences run as they are on hb_block_sparse_fwd."""
    lib = _lib.load()
    B, H, N, D = q.shape
    blocks = N // 64
    stream = _lib.stream_ptr(q.device)
    if blocks <= PAIR_MAX_BLOCKS:
        width = min(2 * kv_indices.shape[1], blocks)
        ids, flags, counts = pair_rows(kv_indices, kv_counts, blocks, 64, width)
        ws = attention_workspace(q.device, B, H, N, D, global_tokens, width, 64, paired=1,
                                 all_queries=all_queries)
        rc = lib.hb_paired_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            lse.data_ptr() if lse is not None else None, _strides(q, k, v, out), B, H, N, D,
            _dtype_code(q), ids.data_ptr(), flags.data_ptr(), counts.data_ptr(), width,
            global_tokens, 64, int(all_queries), scale_log2, ws.data_ptr(), ws.numel(), num_groups,
            stream)
        _lib.check(rc, "hb_paired_fwd")
        return
    width = kv_indices.shape[1]
    ws = attention_workspace(q.device, B, H, N, D, global_tokens, width, 64, paired=0,
                             all_queries=all_queries)
    rc = lib.hb_block_sparse_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        lse.data_ptr() if lse is not None else None, _strides(q, k, v, out), B, H, N, D,
        _dtype_code(q), kv_indices.data_ptr(), kv_counts.data_ptr(), width, global_tokens, 64,
        int(all_queries), scale_log2, ws.data_ptr(), ws.numel(), num_groups, stream)
    _lib.check(rc, "hb_block_sparse_fwd")


@sparse_fwd.register_fake
def _(q, k, v, out, lse, kv_indices, kv_counts, global_tokens, scale_log2, all_queries,
      num_groups):
    return None


@torch.library.custom_op(f"{_NS}::pair_rows", mutates_args=(), device_types=("cuda", "cpu"))
def pair_rows(kv_indices: Tensor, kv_counts: Tensor, total_blocks: int, key_block_size: int,
              paired_width: int) -> tuple[Tensor, Tensor, Tensor]:
    """hb_pair_rows: rows 2r and 2r + 1 of an unpaired table become paired row r (ids, flags with
    bit half + 2*key_half, counts), ascending and zero-padded (paired_metadata.py:26-51); an odd
    row count is paired from the end, paired row 0 holding an empty half 0.  CPU tensors are
    paired by hb_pair_rows_host."""
    from ._tables import pair_rows_device

    return pair_rows_device(kv_indices, kv_counts, total_blocks, key_block_size=key_block_size,
                            paired_width=paired_width)


@pair_rows.register_fake
def _(kv_indices, kv_counts, total_blocks, key_block_size, paired_width):
    prows = (kv_indices.shape[0] + 1) // 2
    ids = kv_indices.new_empty((prows, paired_width))
    return ids, torch.empty_like(ids), kv_indices.new_empty((prows,))


def _gather_shape(x, dim, index):
    shape = list(x.shape)
    shape[dim] = index.shape[0]
    return shape


@torch.library.custom_op(f"{_NS}::gather_rows", mutates_args=(), device_types="cuda")
def gather_rows(x: Tensor, dim: int, index: Tensor) -> Tensor:
    """x.index_select(dim, index) by hb_gather_rows (flux_adapter.py:209-212, :243), bit for bit;
    the dims after ``dim`` must be contiguous (see layout.index_select_rows)."""
    from .layout import gather_into

    return gather_into(x, dim % x.ndim, index)


@gather_rows.register_fake
def _(x, dim, index):
    return x.new_empty(_gather_shape(x, dim % x.ndim, index))
