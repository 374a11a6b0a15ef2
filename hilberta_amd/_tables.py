"""Drives the block-table builder through the C ABI: the HIP kernels of csrc/tables.hip on a
GPU, or their host counterparts (csrc/tables_host.hip, the ``*_host`` entry points, bit-identical)
when the caller asks for ``device="cpu"``.

On the GPU all integer work runs on the device.  The only host synchronisations are the ones the
table format forces at setup time: the number of shared blocks of the layout (it sizes the global
prefix) and the widest row of each emitted table (it is the table width).  The host builder is
for plan setup on machines without a GPU; the attention kernels have no host path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


def _dev(device):
    """The device tables are built on: ``None`` is the current HIP device; ``"cpu"`` selects the
    host builder explicitly (it is never chosen in place of a GPU)."""
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("no HIP device: pass device='cpu' to build the tables on the host")
        return torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    if device.type not in ("cuda", "cpu"):
        raise ValueError("the table builder runs on a HIP device (cuda:N) or on the host (cpu)")
    return device


def _run(device, name, *args):
    """Call entry point ``name`` on ``device``: the HIP launch on the current stream, or its
    ``_host`` counterpart (no stream argument) for CPU tensors."""
    lib = _lib.load()
    if device.type == "cpu":
        rc = getattr(lib, name + "_host")(*args)
    else:
        rc = getattr(lib, name)(*args, _lib.stream_ptr(device))
    _lib.check(rc, name)


@dataclass
class DeviceLayout:
    """Composite Hilbert order and physical packing, resident on the device."""

    grid_size: int
    block_size: int
    text_tokens: int
    shared_blocks: int
    original_order: torch.Tensor
    inverse_original: torch.Tensor
    image_order: torch.Tensor
    inverse_image_order: torch.Tensor
    physical_original_blocks: torch.Tensor
    original_to_physical: torch.Tensor

    @property
    def image_tokens(self):
        return self.grid_size**2

    @property
    def image_blocks(self):
        return self.image_tokens // self.block_size

    @property
    def text_blocks(self):
        return self.text_tokens // self.block_size

    @property
    def global_blocks(self):
        return self.text_blocks + self.shared_blocks

    @property
    def total_blocks(self):
        return self.text_blocks + self.image_blocks

    @property
    def ordinary_blocks(self):
        return self.total_blocks - self.global_blocks

    @property
    def words(self):
        return (self.total_blocks + 31) // 32


def hilbert_order_device(grid_size, device=None):
    device = _dev(device)
    out = torch.empty(grid_size * grid_size, dtype=torch.int64, device=device)
    _run(device, "hb_hilbert_order", grid_size, out.data_ptr())
    return out


def layout_device(grid_size, block_size, text_tokens, shared, device=None):
    device = _dev(device)
    n = grid_size * grid_size
    nb = n // block_size
    i64 = dict(dtype=torch.int64, device=device)
    t = [torch.empty(n, **i64) for _ in range(4)] + [torch.empty(nb, **i64) for _ in range(2)]
    status = torch.zeros(3, dtype=torch.int32, device=device)
    _run(device, "hb_plan_layout", grid_size, block_size, text_tokens, int(bool(shared)),
         *[x.data_ptr() for x in t], status.data_ptr())
    # setup-time sync: the prefix length is data dependent; the same read checks that the image
    # order is a permutation, so the per-forward gathers may trust it
    n_shared, partial, bad_order = status.tolist()
    if partial:
        raise ValueError("Shared square must be a union of complete original blocks")
    if bad_order:
        raise RuntimeError("hb_plan_layout produced an image order that is not a permutation")
    return DeviceLayout(grid_size, block_size, text_tokens, n_shared, *t)


def phase_bits_device(layout: DeviceLayout, tile_count, phase, bridge_mode, k, scratch=None):
    """Adjacency bitmap [ordinary, words] (int32 storage of uint32 words) and chosen bridges [nb, k]."""
    device = layout.original_order.device
    kk = max(int(k), 1)
    bits = torch.empty((layout.ordinary_blocks, layout.words), dtype=torch.int32, device=device)
    chosen = torch.full((layout.image_blocks, kk), -1, dtype=torch.int64, device=device)
    if bridge_mode and scratch is None:
        scratch = torch.empty(layout.image_blocks**2, dtype=torch.int32, device=device)
    _run(device, "hb_plan_phase_bits",
         layout.inverse_original.data_ptr(), layout.physical_original_blocks.data_ptr(),
         layout.original_to_physical.data_ptr(), layout.grid_size, tile_count, layout.text_tokens,
         layout.block_size, layout.shared_blocks, phase, bridge_mode, kk,
         scratch.data_ptr() if bridge_mode else None, chosen.data_ptr(), bits.data_ptr())
    return bits, chosen


def _bits_counts(bits, total_blocks, unpaired, paired, key_block_size):
    """Row counts (unpaired and/or paired) of a bitmap and the widest rows, on the device."""
    device = bits.device
    rows = bits.shape[0]
    i32 = dict(dtype=torch.int32, device=device)
    counts = torch.empty(rows, **i32) if unpaired else None
    pcounts = torch.empty(rows // 2, **i32) if paired else None
    maxc = torch.zeros(2, **i32)
    _run(device, "hb_bits_counts", bits.data_ptr(), rows, total_blocks, key_block_size,
         counts.data_ptr() if unpaired else None, pcounts.data_ptr() if paired else None,
         maxc.data_ptr())
    return counts, pcounts, maxc


def _bits_emit(bits, total_blocks, counts, pcounts, width, pwidth, unpaired, paired,
               key_block_size):
    """Ascending tables of a bitmap at the given widths (rows zero-padded)."""
    device = bits.device
    rows = bits.shape[0]
    i32 = dict(dtype=torch.int32, device=device)
    ids = torch.empty((rows, width), **i32) if unpaired else None
    pids = torch.empty((rows // 2, pwidth), **i32) if paired else None
    pflags = torch.empty((rows // 2, pwidth), **i32) if paired else None
    _run(device, "hb_bits_emit", bits.data_ptr(), rows, total_blocks, key_block_size,
         ids.data_ptr() if unpaired else None, width, pids.data_ptr() if paired else None,
         pflags.data_ptr() if paired else None, pwidth)
    out = {}
    if unpaired:
        out.update(kv_indices=ids, kv_counts=counts)
    if paired:
        out.update(paired_indices=pids, paired_flags=pflags, paired_counts=pcounts)
    return out


def emit_device(bits, total_blocks, *, unpaired=True, paired=False, key_block_size=64,
                paired_width=None):
    """Tables from a bitmap: returns dict with ids/counts and/or paired ids/flags/counts (device).

    The table widths are the widest rows, read back to the host (one synchronisation), unless only
    paired tables are asked for with ``paired_width`` given: an upper bound on the paired row
    length, used as is (rows zero-padded to it), with no host synchronisation.
    """
    counts, pcounts, maxc = _bits_counts(bits, total_blocks, unpaired, paired, key_block_size)
    if paired_width is not None and not unpaired:
        width, pwidth = 1, int(paired_width)
    else:
        width, pwidth = (max(x, 1) for x in maxc.tolist())  # setup-time sync: table widths
    return _bits_emit(bits, total_blocks, counts, pcounts, width, pwidth, unpaired, paired,
                      key_block_size)


def emit_device_many(bits_list, total_blocks, *, unpaired=True, paired=False, key_block_size=64):
    """emit_device over several bitmaps (the phases of a plan) with one host synchronisation for
    all their table widths: every count launch is queued before the widths are read back, so the
    device runs the phases back to back instead of draining between them."""
    counted = [_bits_counts(b, total_blocks, unpaired, paired, key_block_size) for b in bits_list]
    widths = torch.stack([m for _, _, m in counted]).tolist()  # setup-time sync: table widths
    return [
        _bits_emit(b, total_blocks, c, pc, max(w[0], 1), max(w[1], 1), unpaired, paired,
                   key_block_size)
        for b, (c, pc, _), w in zip(bits_list, counted, widths)
    ]


def _check_table(kv_indices, kv_counts):
    """The entry points read ``kv_indices`` as int32 [rows, width] and ``kv_counts`` as int32
    [rows], contiguous, on one device."""
    if (kv_indices.dtype != torch.int32 or kv_counts.dtype != torch.int32 or kv_indices.dim() != 2
            or kv_counts.shape != (kv_indices.shape[0],) or not kv_indices.is_contiguous()
            or not kv_counts.is_contiguous() or kv_indices.device != kv_counts.device):
        raise ValueError("tables must be contiguous int32 kv_indices [rows, width] and kv_counts "
                         "[rows] on one device")


def table_bits_device(kv_indices, kv_counts, total_blocks):
    _check_table(kv_indices, kv_counts)
    device = kv_indices.device
    rows, width = kv_indices.shape
    words = (total_blocks + 31) // 32
    bits = torch.empty((rows, words), dtype=torch.int32, device=device)
    _run(device, "hb_table_bits", kv_indices.data_ptr(), kv_counts.data_ptr(), rows, width,
         total_blocks, bits.data_ptr())
    return bits


def pair_rows_device(kv_indices, kv_counts, total_blocks, *, key_block_size=64, paired_width,
                     overflow=None):
    """Pair an unpaired device table in one launch, without a host synchronisation.

    The device form of ``pair_metadata`` (reference hilberta/paired_metadata.py:26-51): rows 2r
    and 2r + 1 become paired row r (an odd row count is paired from the end: rows 2r - 1 and 2r,
    paired row 0 with an empty half 0), ascending, flag bit (half + 2*key_half), zero-padded to
    ``paired_width``, which should bound every paired row's entry count (min(2 * width, key
    blocks) always does).  ``overflow`` may be a device int32 scalar tensor that is set to 1 when
    some paired row had to be cut to ``paired_width`` entries.  Returns (ids, flags, counts) as
    int32 device tensors.  CPU tables are paired on the host (hb_pair_rows_host).
    """
    _check_table(kv_indices, kv_counts)
    device = kv_indices.device
    rows, width = kv_indices.shape
    prows = (rows + 1) // 2
    ids = torch.empty((prows, paired_width), dtype=torch.int32, device=device)
    flags = torch.empty_like(ids)
    counts = torch.empty((prows,), dtype=torch.int32, device=device)
    _run(device, "hb_pair_rows", kv_indices.data_ptr(), kv_counts.data_ptr(), rows, width,
         total_blocks, key_block_size, ids.data_ptr(), flags.data_ptr(), counts.data_ptr(),
         paired_width, overflow.data_ptr() if overflow is not None else None)
    return ids, flags, counts


def quad_rows_device(kv_indices, kv_counts, total_blocks, *, kv_flags=None, quad_width,
                     overflow=None):
    """Quad tables for the 256-query kernel (hb_quad_fwd) in one launch, without a host sync.

    With ``kv_flags``: paired 64-key tables (``pair_metadata``'s output, reference
    hilberta/paired_metadata.py:26-51); quad row r is the union of paired rows 2r and 2r + 1 with
    flag bit 2j + half from paired row 2r + j.  Without: unpaired tables, quad row r the union of
    rows 4r .. 4r + 3 with flag bit j from row 4r + j.  Rows are ascending, zero padded to
    ``quad_width`` (min(2 * paired width, key blocks) always bounds them); ``overflow`` as in
    pair_rows_device.  Returns (ids, flags, counts) as int32 device tensors.
    """
    _lib.require_gpu(kv_indices, kv_counts)
    device = kv_indices.device
    rows, width = kv_indices.shape
    group = 2 if kv_flags is not None else 4
    ids = torch.empty((rows // group, quad_width), dtype=torch.int32, device=device)
    flags = torch.empty_like(ids)
    counts = torch.empty((rows // group,), dtype=torch.int32, device=device)
    rc = _lib.load().hb_quad_rows(kv_indices.data_ptr(),
                                  kv_flags.data_ptr() if kv_flags is not None else None,
                                  kv_counts.data_ptr(), rows, width, total_blocks, ids.data_ptr(),
                                  flags.data_ptr(), counts.data_ptr(), quad_width,
                                  overflow.data_ptr() if overflow is not None else None,
                                  _lib.stream_ptr(device))
    _lib.check(rc, "hb_quad_rows")
    return ids, flags, counts


def paired_plan_tables_device(grid_size, tile_count, k, text_tokens, shared, key_block_size,
                              device=None):
    """Layout and the four phases' paired tables of bridge_k_plan + pair_metadata in six launches
    and one host read (hb_paired_plan_tables / hb_paired_plan_emit).

    Returns (DeviceLayout, [(ids, flags, counts) per phase]) on the device.  The host read takes the
    shared-prefix length, the layout checks and the four table widths at once.  With
    ``device="cpu"`` the same tables come from the host builder (_paired_plan_tables_host).
    """
    import ctypes

    device = _dev(device)
    if device.type == "cpu":
        return _paired_plan_tables_host(grid_size, tile_count, k, text_tokens, shared,
                                        key_block_size)
    lib = _lib.load()
    n = grid_size * grid_size
    nb = n // 64
    orders = torch.empty(4 * n + 2 * nb, dtype=torch.int64, device=device)
    t = [orders[i * n:(i + 1) * n] for i in range(4)]
    t += [orders[4 * n:4 * n + nb], orders[4 * n + nb:]]
    need = lib.hb_paired_plan_scratch_bytes(grid_size, text_tokens)
    if need < 0:
        raise ValueError("invalid plan geometry")
    scratch = torch.empty(need, dtype=torch.uint8, device=device)
    status = torch.empty(7, dtype=torch.int32, device=device)
    stream = _lib.stream_ptr(device)
    rc = lib.hb_paired_plan_tables(grid_size, tile_count, k, text_tokens, int(bool(shared)),
                                   key_block_size, *[x.data_ptr() for x in t], scratch.data_ptr(),
                                   status.data_ptr(), stream)
    _lib.check(rc, "hb_paired_plan_tables")
    # setup-time sync: the shared-prefix length, the layout checks and the table widths
    n_shared, partial, bad_order, *widths = status.tolist()
    if partial:
        raise ValueError("Shared square must be a union of complete original blocks")
    if bad_order:
        raise RuntimeError("hb_paired_plan_tables produced an image order that is not a permutation")
    layout = DeviceLayout(grid_size, 64, text_tokens, n_shared, *t)
    nq = nb - n_shared
    if nq % 2:
        raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
    rows = nq // 2
    widths = [max(int(w), 1) for w in widths]
    buf = torch.empty(sum(2 * rows * w + rows for w in widths), dtype=torch.int32, device=device)
    tables, off = [], 0
    for w in widths:
        ids = buf[off:off + rows * w].view(rows, w)
        flags = buf[off + rows * w:off + 2 * rows * w].view(rows, w)
        counts = buf[off + 2 * rows * w:off + 2 * rows * w + rows]
        off += 2 * rows * w + rows
        tables.append((ids, flags, counts))
    ptrs = lambda i: (ctypes.c_void_p * 4)(*[tb[i].data_ptr() for tb in tables])  # noqa: E731
    rc = lib.hb_paired_plan_emit(grid_size, text_tokens, n_shared, key_block_size, scratch.data_ptr(),
                                 ptrs(0), ptrs(1), ptrs(2), (ctypes.c_int32 * 4)(*widths), stream)
    _lib.check(rc, "hb_paired_plan_emit")
    return layout, tables


def _paired_plan_tables_host(grid_size, tile_count, k, text_tokens, shared, key_block_size):
    """paired_plan_tables_device on the host: the layout, each phase's reciprocal top-K bitmap and
    its paired tables from the host entry points, the steps the fused device plan runs."""
    cpu = torch.device("cpu")
    layout = layout_device(grid_size, 64, text_tokens, shared, cpu)
    if layout.ordinary_blocks % 2:
        raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
    scratch = torch.empty(layout.image_blocks**2, dtype=torch.int32)
    bits = [phase_bits_device(layout, tile_count, phase, 2, k, scratch)[0] for phase in range(4)]
    tables = emit_device_many(bits, layout.total_blocks, unpaired=False, paired=True,
                              key_block_size=key_block_size)
    return layout, [(t["paired_indices"], t["paired_flags"], t["paired_counts"]) for t in tables]
