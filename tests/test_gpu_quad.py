"""GPU: 256-query quad items.  The quad table builder (hb_quad_rows) is bit-exact against a
numpy union of the paired (or unpaired) rows; the quad kernel (hb_quad_fwd) gives ordinary rows
bitwise equal to the paired kernel's (every query sees the same key blocks in the same order with
the same arithmetic; blocks another query block needs are masked to exact zeros), and global rows
within the fp32 oracle's tolerance."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as A
from tests.helpers import compare, device_paired, oracle_paired, oracle_plan, reference, say

pytestmark = pytest.mark.gpu
D = 128
SCALE_LOG2 = D**-0.5 * 1.4426950408889634


def _union(ids, flags, counts, group, bits):
    """Quad rows by a plain numpy loop: per row group, key block -> OR of shifted flags."""
    out = []
    for r in range(len(counts) // group):
        d = {}
        for j in range(group):
            row = group * r + j
            for e in range(counts[row]):
                f = 1 if flags is None else int(flags[row, e]) & 3
                d[int(ids[row, e])] = d.get(int(ids[row, e]), 0) | (f << (bits * j))
        out.append(sorted(d.items()))
    return out


def _check_quads(qi, qf, qc, expect, width):
    qi, qf, qc = (x.cpu().numpy() for x in (qi, qf, qc))
    assert qi.shape == (len(expect), width)
    for r, row in enumerate(expect):
        n = len(row)
        assert qc[r] == n, f"row {r}: count {qc[r]} != {n}"
        assert qi[r, :n].tolist() == [k for k, _ in row], f"row {r} ids"
        assert qf[r, :n].tolist() == [f for _, f in row], f"row {r} flags"
        assert not qi[r, n:].any() and not qf[r, n:].any(), f"row {r} padding"


@pytest.mark.parametrize("name", ["1024_t4k1", "1024_t16k3", "2048_t16k3"])
@pytest.mark.parametrize("phase", [0, 3])
def test_quad_rows_from_paired_and_unpaired(hip_device, name, phase):
    from hilberta_amd._tables import quad_rows_device

    say(f"case quad_rows {name} phase {phase}")
    plan = oracle_plan(name)
    T = plan["total_tokens"] // 64
    pm = oracle_paired(plan, phase)
    meta = device_paired(pm, hip_device)
    width = min(2 * meta.kv_indices.shape[1], T)
    ov = torch.zeros(1, dtype=torch.int32, device=hip_device)
    qi, qf, qc = quad_rows_device(meta.kv_indices, meta.kv_counts, T, kv_flags=meta.kv_flags,
                                  quad_width=width, overflow=ov)
    expect = _union(pm["kv_indices"], pm["kv_flags"], pm["kv_counts"], 2, 2)
    _check_quads(qi, qf, qc, expect, width)
    assert ov.item() == 0
    # from the unpaired rows directly: the same tables
    p = plan["phases"][phase]
    ids = torch.from_numpy(p["kv_indices"]).to(hip_device)
    counts = torch.from_numpy(p["kv_counts"]).to(hip_device)
    ui, uf, uc = quad_rows_device(ids, counts, T, quad_width=width)
    for a, b in ((ui, qi), (uf, qf), (uc, qc)):
        assert torch.equal(a, b)


def test_quad_rows_reports_overflow(hip_device):
    from hilberta_amd._tables import quad_rows_device

    plan = oracle_plan("1024_t16k3")
    meta = device_paired(oracle_paired(plan, 1), hip_device)
    T = plan["total_tokens"] // 64
    ov = torch.zeros(1, dtype=torch.int32, device=hip_device)
    qi, qf, qc = quad_rows_device(meta.kv_indices, meta.kv_counts, T, kv_flags=meta.kv_flags,
                                  quad_width=4, overflow=ov)
    assert ov.item() == 1 and int(qc.max()) == 4


def _run(lib, fn, q, k, v, ids, flags, counts, G, kind):
    B, H, N, _ = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(B, H, N, dtype=torch.float32, device=q.device)
    need = lib.hb_attention_workspace_bytes(B, H, N, D, G, ids.shape[1], 64, kind, 1)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=q.device)
    strides = (ctypes.c_int64 * 12)(*[s for x in (q, k, v, out) for s in x.stride()[:3]])
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(), strides, B, H,
            N, D, 0, ids.data_ptr(), flags.data_ptr(), counts.data_ptr(), ids.shape[1], G]
    if kind == 1:
        args.append(64)
    args += [1, SCALE_LOG2, ws.data_ptr(), ws.numel(), 0, torch.cuda.current_stream().cuda_stream]
    rc = getattr(lib, fn)(*args)
    assert rc == 0, lib.hb_last_error()
    return out, lse


@pytest.mark.parametrize("name,phase,batch,bnhd", [("1024_t16k3", 1, 1, False),
                                                   ("1024_t4k1", 2, 2, True),
                                                   ("2048_t16k3", 0, 1, False)])
def test_quad_fwd_matches_paired_kernel(hip_device, name, phase, batch, bnhd):
    from hilberta_amd import _lib
    from hilberta_amd._tables import quad_rows_device

    say(f"case quad_fwd {name} phase {phase} B={batch} bnhd={bnhd}")
    lib = _lib.load()
    plan = oracle_plan(name)
    N, G = plan["total_tokens"], plan["global_tokens"]
    heads = 4
    q, k, v = A.seeded_qkv(batch, heads, N, D, seed=41)
    if bnhd:
        q, k, v = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    q, k, v = (x.to(hip_device) for x in (q, k, v))
    meta = device_paired(oracle_paired(plan, phase), hip_device)
    T = N // 64
    qi, qf, qc = quad_rows_device(meta.kv_indices, meta.kv_counts, T, kv_flags=meta.kv_flags,
                                  quad_width=min(2 * meta.kv_indices.shape[1], T))
    o_p, l_p = _run(lib, "hb_paired_fwd", q, k, v, meta.kv_indices, meta.kv_flags, meta.kv_counts,
                    G, 1)
    o_q, l_q = _run(lib, "hb_quad_fwd", q, k, v, qi, qf, qc, G, 2)
    torch.cuda.synchronize()
    assert torch.equal(o_q[:, :, G:], o_p[:, :, G:]), "ordinary rows differ from the paired kernel"
    assert torch.equal(l_q[:, :, G:], l_p[:, :, G:]), "ordinary LSE differs from the paired kernel"
    ref_o, ref_l = reference(q.cpu(), k.cpu(), v.cpu(), plan, phase)
    compare(o_q, l_q, ref_o, ref_l, f"quad {name} global rows", rows=slice(0, G))
