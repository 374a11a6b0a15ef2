"""Hilbert ordering and grid neighbours (drop-in for reference hilberta/geometry.py).

``hilbert_order`` is computed on the GPU (hb_hilbert_order: d2xy Hilbert then a vertical flip to
raster ids (g-1-y)*g + x, geometry.py:6-25), or on the host with ``device="cpu"``
(hb_hilbert_order_host), and returned on the CPU like the reference's.
``neighbor_pairs`` is host bookkeeping (the device builder enumerates the same pairs inside its
score kernel): ascending undirected 4/8-neighbour pairs, row-major, right then down (then the two
diagonals), geometry.py:28-43.
"""

from __future__ import annotations

import torch

from ._tables import hilbert_order_device


def hilbert_order(grid_size=64, *, device=None):
    if grid_size < 2 or grid_size & (grid_size - 1):
        raise ValueError("Hilbert grid side must be a power of two >= 2")
    return hilbert_order_device(int(grid_size), device).cpu()


def neighbor_pairs(grid_size, connectivity=4):
    if int(grid_size) != grid_size or grid_size < 1 or connectivity not in (4, 8):
        raise ValueError("positive integer grid_size and connectivity 4 or 8 required")
    g = int(grid_size)
    directions = [(0, 1), (1, 0)] + ([(1, 1), (1, -1)] if connectivity == 8 else [])
    y, x = torch.meshgrid(torch.arange(g), torch.arange(g), indexing="ij")
    first, second, valid = [], [], []
    for dy, dx in directions:
        ny, nx = y + dy, x + dx
        valid.append((ny >= 0) & (ny < g) & (nx >= 0) & (nx < g))
        first.append(y * g + x)
        second.append(ny * g + nx)
    keep = torch.stack(valid, -1).reshape(-1)
    a = torch.stack(first, -1).reshape(-1)[keep]
    b = torch.stack(second, -1).reshape(-1)[keep]
    return torch.stack((a, b), 1).to(torch.long)
