"""hb_paired_fwd_noalloc: the paired forward on the library's static scratch, through the C ABI.

Two calls in a row, the second with smaller shapes (fewer heads, a shorter sequence, no split
global tiles), each against hb_paired_fwd with a caller workspace on the same inputs: the same
kernels on the same plan, so the outputs and LSE are equal bit for bit, and both are within the
suite's tolerance of the fp32 oracle.  The first call splits its global query tiles, so the split
partials and the merge run out of the static scratch too.  A ragged case follows: tables paired
on the device from an odd row count with a global prefix that is an odd multiple of 64, so both
kinds of overhanging half are skipped with the partials in the static scratch.
"""

import ctypes

import pytest
import torch

from oracle import attention as A
from tests.helpers import compare, device_paired, oracle_paired, oracle_plan, reference, say

pytestmark = pytest.mark.gpu

D = 128


def _args(q, k, v, out, lse, meta):
    from hilberta_amd.sparse_kernel import LOG2E, _strides

    B, H, N, Dh = q.shape
    strides = (ctypes.c_int64 * 12)(*_strides(q, k, v, out))
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(), strides, B, H,
            N, Dh, 0, meta.kv_indices.data_ptr(), meta.kv_flags.data_ptr(),
            meta.kv_counts.data_ptr(), meta.kv_indices.shape[1], meta.global_tokens,
            meta.key_block_size, 1, Dh**-0.5 * LOG2E)


def _both(q, k, v, meta):
    from hilberta_amd import _lib

    lib = _lib.load()
    B, H, N, Dh = q.shape
    width = meta.kv_indices.shape[1]
    need = lib.hb_attention_workspace_bytes(B, H, N, Dh, meta.global_tokens, width,
                                            meta.key_block_size, 1, 1)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=q.device)
    stream = _lib.stream_ptr(q.device)
    out_ws, out_na = torch.empty_like(q), torch.empty_like(q)
    lse_ws = torch.empty(B, H, N, dtype=torch.float32, device=q.device)
    lse_na = torch.empty_like(lse_ws)
    rc = lib.hb_paired_fwd(*_args(q, k, v, out_ws, lse_ws, meta), ws.data_ptr(), ws.numel(), 0, stream)
    _lib.check(rc, "hb_paired_fwd")
    rc = lib.hb_paired_fwd_noalloc(*_args(q, k, v, out_na, lse_na, meta), 0, stream)
    _lib.check(rc, "hb_paired_fwd_noalloc")
    torch.cuda.synchronize()
    return need, (out_ws, lse_ws), (out_na, lse_na)


def test_noalloc_matches_workspace_entry_point(hip_device):
    cases = [("2048_t16k3", 0, 6), ("1024_t4k1", 2, 2)]  # the second call is smaller
    for name, phase, heads in cases:
        plan = oracle_plan(name)
        q, k, v = A.seeded_qkv(1, heads, plan["total_tokens"], D, seed=23)
        qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
        meta = device_paired(oracle_paired(plan, phase), hip_device)
        say(f"case noalloc {name} phase {phase} heads={heads}")
        need, (o_ws, l_ws), (o_na, l_na) = _both(qd, kd, vd, meta)
        if name == "2048_t16k3":
            assert need > 256, "the first call must use split partials"
        assert torch.equal(o_na, o_ws), f"{name}: output differs from hb_paired_fwd"
        assert torch.equal(l_na, l_ws), f"{name}: LSE differs from hb_paired_fwd"
        if name == "1024_t4k1":
            ref_o, ref_l = reference(q, k, v, plan, phase)
            compare(o_na.cpu(), l_na.cpu(), ref_o, ref_l, f"noalloc {name}")
        else:
            G = plan["global_tokens"]
            qf, kf, vf = qd.float(), kd.float(), vd.float()
            s = torch.matmul(qf[:, :, :G], kf.transpose(-1, -2).contiguous()) * D**-0.5
            compare(o_na[:, :, :G], l_na[:, :, :G], torch.matmul(torch.softmax(s, -1), vf),
                    torch.logsumexp(s, -1), f"noalloc {name} global rows")


def test_noalloc_ragged_matches_workspace_entry_point(hip_device):
    import numpy as np
    from types import SimpleNamespace

    from hilberta_amd._tables import pair_rows_device

    G, rows, heads = 576, 71, 4
    N = G + 64 * rows
    T_ = N // 64
    rng = np.random.default_rng(47)
    width = G // 64 + 6
    ids = np.zeros((rows, width), np.int32)
    counts = np.zeros(rows, np.int32)
    for r in range(rows):
        extra = rng.choice(np.arange(G // 64, T_), size=rng.integers(1, 7), replace=False)
        row = np.concatenate([np.arange(G // 64), np.sort(extra)]).astype(np.int32)
        ids[r, :len(row)] = row
        counts[r] = len(row)
    pid, pfl, pct = pair_rows_device(torch.from_numpy(ids).to(hip_device),
                                     torch.from_numpy(counts).to(hip_device), T_,
                                     paired_width=min(2 * width, T_))
    meta = SimpleNamespace(kv_indices=pid, kv_flags=pfl, kv_counts=pct, global_tokens=G,
                           key_block_size=64)
    q, k, v = A.seeded_qkv(1, heads, N, D, seed=29)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    say(f"case noalloc ragged G={G} rows={rows}")
    need, (o_ws, l_ws), (o_na, l_na) = _both(qd, kd, vd, meta)
    assert need > 256, "the global tiles must split"
    assert torch.equal(o_na, o_ws) and torch.equal(l_na, l_ws), "differs from hb_paired_fwd"
    ref_o, ref_l = A.block_sparse_attention(q, k, v, ids, counts, global_tokens=G)
    compare(o_na.cpu(), l_na.cpu(), ref_o, ref_l, "noalloc ragged")
