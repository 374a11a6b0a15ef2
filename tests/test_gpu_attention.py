"""GPU parity of the HIP block-sparse attention against the fp32 oracle (tolerance in helpers.py).

Inputs: Q/K/V drawn on the CPU from seed 2707 (q, k, v order, fp32 -> bf16), tables from the CPU
oracle.  The fp32 reference runs on the CPU where it takes seconds (1024 px) and, for the 2048 px
shapes, as the same torch fp32 code on the device over every query row.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import topology as T
from tests.helpers import (
    compare,
    device_paired,
    oracle_paired,
    oracle_plan,
    reference,
    say,
)

pytestmark = pytest.mark.gpu

H, D = 24, 128


def _qkv(plan, batch=1, heads=H, dim=D, dtype=torch.bfloat16, seed=2707):
    return A.seeded_qkv(batch, heads, plan["total_tokens"], dim, seed=seed, dtype=dtype)


@pytest.mark.parametrize("name", ["1024_t4k1", "1024_t16k3"])
def test_paired_1024_all_phases(hip_device, name):
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan(name)
    q, k, v = _qkv(plan)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    for phase in range(4):
        say(f"case paired {name} phase {phase} B=1")
        meta = device_paired(oracle_paired(plan, phase), hip_device)
        lse = torch.empty(q.shape[:3], dtype=torch.float32, device=hip_device)
        out = paired_attention(qd, kd, vd, meta, global_strategy="triton", num_warps=8, lse=lse)
        torch.cuda.synchronize()
        ref_o, ref_l = reference(q, k, v, plan, phase)
        compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"{name} phase {phase}")


def test_paired_batch4_bnhd_views(hip_device):
    """B=4 with the adapter's BNHD storage viewed as BHND and a caller-provided BNHD output."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t4k1")
    N = plan["total_tokens"]
    q, k, v = _qkv(plan, batch=4)
    say("case paired 1024_t4k1 B=4 BNHD")
    to_bnhd = lambda x: x.transpose(1, 2).contiguous().to(hip_device).transpose(1, 2)  # noqa: E731
    qd, kd, vd = to_bnhd(q), to_bnhd(k), to_bnhd(v)
    assert qd.stride() == (N * H * D, D, H * D, 1)
    out = torch.empty(4, N, H, D, dtype=torch.bfloat16, device=hip_device).transpose(1, 2)
    meta = device_paired(oracle_paired(plan, 2), hip_device)
    res = paired_attention(qd, kd, vd, meta, out=out)
    assert res is out
    torch.cuda.synchronize()
    ref_o, ref_l = reference(q, k, v, plan, 2)
    compare(out.cpu(), None, ref_o, ref_l, "1024_t4k1 B=4 BNHD")


def test_paired_key_block_128(hip_device):
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t16k3")
    q, k, v = _qkv(plan, heads=4)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    for phase in (0, 1):
        say(f"case paired KB128 1024_t16k3 phase {phase}")
        meta = device_paired(oracle_paired(plan, phase, key_block_size=128), hip_device)
        lse = torch.empty(q.shape[:3], dtype=torch.float32, device=hip_device)
        out = paired_attention(qd, kd, vd, meta, lse=lse)
        torch.cuda.synchronize()
        ref_o, ref_l = reference(q, k, v, plan, phase)
        compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"KB128 phase {phase}")


def test_unpaired_sparse_attention(hip_device):
    from hilberta_amd.sparse_kernel import sparse_attention

    plan = oracle_plan("1024_t16k3")
    q, k, v = _qkv(plan, heads=6)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    for phase in range(4):
        say(f"case unpaired 1024_t16k3 phase {phase}")
        p = plan["phases"][phase]
        ids = torch.from_numpy(p["kv_indices"]).to(hip_device)
        counts = torch.from_numpy(p["kv_counts"]).to(hip_device)
        lse = torch.empty(q.shape[:3], dtype=torch.float32, device=hip_device)
        out = sparse_attention(qd, kd, vd, ids, counts, global_tokens=plan["global_tokens"], lse=lse)
        torch.cuda.synchronize()
        ref_o, ref_l = reference(q, k, v, plan, phase)
        compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"unpaired phase {phase}")


def _unpaired_kernel(q, k, v, ids, counts, global_tokens, scale):
    """The 64-query-row kernel itself (hb_block_sparse_fwd through the C ABI), output and LSE."""
    import ctypes
    import math as m

    from hilberta_amd import _lib
    from hilberta_amd._workspace import attention_workspace
    from hilberta_amd.sparse_kernel import _strides

    lib = _lib.load()
    B, H, N, Dh = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    width = ids.shape[1]
    ws = attention_workspace(q.device, B, H, N, Dh, global_tokens, width, 64, paired=0, all_queries=1)
    strides = (ctypes.c_int64 * 12)(*_strides(q, k, v, out))
    rc = lib.hb_block_sparse_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                 strides, B, H, N, Dh, 0, ids.data_ptr(), counts.data_ptr(), width,
                                 global_tokens, 64, 1, scale * 1.4426950408889634, ws.data_ptr(),
                                 ws.numel(), 0, _lib.stream_ptr(q.device))
    _lib.check(rc, "hb_block_sparse_fwd")
    return out, lse


def test_unpaired_tables_run_paired(hip_device):
    """sparse_attention pairs 64-query rows on the device and runs the paired kernel: every
    ordinary query row equals the unpaired kernel's bit for bit (same blocks, same order, same
    arithmetic; the other half's blocks add exact zeros); the global rows, chunked differently,
    agree within the suite's tolerance."""
    from hilberta_amd.sparse_kernel import sparse_attention

    plan = oracle_plan("1024_t16k3")
    G = plan["global_tokens"]
    q, k, v = _qkv(plan, heads=4, seed=21)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    for phase in (1, 2):
        say(f"case unpaired tables via the paired kernel, 1024_t16k3 phase {phase}")
        p = plan["phases"][phase]
        ids = torch.from_numpy(p["kv_indices"]).to(hip_device)
        counts = torch.from_numpy(p["kv_counts"]).to(hip_device)
        lse = torch.empty(q.shape[:3], dtype=torch.float32, device=hip_device)
        out = sparse_attention(qd, kd, vd, ids, counts, global_tokens=G, lse=lse)
        ref_o, ref_l = _unpaired_kernel(qd, kd, vd, ids, counts, G, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out[:, :, G:], ref_o[:, :, G:]), "ordinary rows differ"
        assert torch.equal(lse[:, :, G:], ref_l[:, :, G:]), "ordinary LSE differs"
        # the global rows are split into chunks differently, so P is rounded to bf16 against
        # different running maxima: equal to the suite's tolerance, not bit for bit
        assert (out[:, :, :G].float() - ref_o[:, :, :G].float()).abs().max().item() <= 4e-3
        assert (lse[:, :, :G] - ref_l[:, :, :G]).abs().max().item() <= 1e-3


def _random_rows(G, rows, seed, max_extra=7):
    """Random valid unpaired tables: every row holds the global prefix plus 1..max_extra-1 other
    key blocks, ascending."""
    T_ = G // 64 + rows
    rng = np.random.default_rng(seed)
    width = G // 64 + max_extra
    ids = np.zeros((rows, width), np.int32)
    counts = np.zeros(rows, np.int32)
    for r in range(rows):
        size = rng.integers(1, min(max_extra, T_ - G // 64 + 1))
        extra = rng.choice(np.arange(G // 64, T_), size=size, replace=False)
        row = np.concatenate([np.arange(G // 64), np.sort(extra)]).astype(np.int32)
        ids[r, :len(row)] = row
        counts[r] = len(row)
    return ids, counts


@pytest.mark.parametrize("G,rows,dim", [
    (512, 9, 128),   # odd row count: paired row 0 reaches 64 queries into the global prefix
    (576, 8, 128),   # G an odd multiple of 64: the last global tile reaches 64 queries past G
    (576, 9, 64),    # both
    (0, 7, 128),     # no prefix and an odd row count: the empty half lies before token 0
    (64, 5, 128),    # one global 64-query row
    (576, 71, 128),  # 80 key blocks: the global tiles split, merge_kernel skips the overhang
])
def test_ragged_tables_run_paired(hip_device, G, rows, dim):
    """Tables whose 64-query rows do not pair evenly (an odd row count, or a global prefix that is
    an odd multiple of 64) are paired from the end on the device and run on the paired kernel:
    every row against the fp32 oracle, and the ordinary rows bit for bit equal to the unpaired
    64-query-row kernel's (same blocks, same order, same arithmetic)."""
    from hilberta_amd.sparse_kernel import sparse_attention

    N = G + 64 * rows
    ids, counts = _random_rows(G, rows, seed=5 + rows + G)
    q, k, v = A.seeded_qkv(1, 3, N, dim, seed=8)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    say(f"case ragged tables G={G} rows={rows} D={dim} N={N}")
    idd, cnd = torch.from_numpy(ids).to(hip_device), torch.from_numpy(counts).to(hip_device)
    lse = torch.full(q.shape[:3], float("nan"), dtype=torch.float32, device=hip_device)
    out = torch.full_like(qd, float("nan"))
    sparse_attention(qd, kd, vd, idd, cnd, global_tokens=G, lse=lse, out=out)
    torch.cuda.synchronize()
    ref_o, ref_l = A.block_sparse_attention(q, k, v, ids, counts, global_tokens=G)
    compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"ragged G={G} rows={rows}")
    if dim == 128:
        uo, ul = _unpaired_kernel(qd, kd, vd, idd, cnd, G, dim ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out[:, :, G:], uo[:, :, G:]), "ordinary rows differ from the unpaired kernel"
        assert torch.equal(lse[:, :, G:], ul[:, :, G:]), "ordinary LSE differs from the unpaired kernel"


def test_long_ragged_table_runs_paired(hip_device):
    """A ragged table of 4008 key blocks (beyond the old 2048-block pairing limit, N = 256448):
    sparse_attention pairs it on the device; its ordinary rows equal the 64-query kernel's bit for
    bit and its global rows match fp32 attention over every key."""
    from hilberta_amd.sparse_kernel import sparse_attention

    G, rows, dim = 576, 3999, 64
    N = G + 64 * rows
    ids, counts = _random_rows(G, rows, seed=61)
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 1, N, dim, seed=62))
    idd, cnd = torch.from_numpy(ids).to(hip_device), torch.from_numpy(counts).to(hip_device)
    say(f"case long ragged table N={N} D={dim}")
    lse = torch.empty(1, 1, N, dtype=torch.float32, device=hip_device)
    out = sparse_attention(q, k, v, idd, cnd, global_tokens=G, lse=lse)
    uo, ul = _unpaired_kernel(q, k, v, idd, cnd, G, dim ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out[:, :, G:], uo[:, :, G:]), "ordinary rows differ from the unpaired kernel"
    assert torch.equal(lse[:, :, G:], ul[:, :, G:]), "ordinary LSE differs from the unpaired kernel"
    s = torch.matmul(q[:, :, :G].float(), k.float().transpose(-1, -2).contiguous()) * dim ** -0.5
    compare(out[:, :, :G], lse[:, :, :G], torch.matmul(torch.softmax(s, -1), v.float()),
            torch.logsumexp(s, -1), "long ragged global rows")


@pytest.mark.parametrize("dtype,dim", [(torch.float16, 128), (torch.bfloat16, 64), (torch.float16, 64)])
def test_dtypes_and_head_dim(hip_device, dtype, dim):
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t16k3")
    q, k, v = _qkv(plan, heads=3, dim=dim, dtype=dtype, seed=11)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    say(f"case paired dtype={dtype} D={dim}")
    meta = device_paired(oracle_paired(plan, 3), hip_device)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=hip_device)
    out = paired_attention(qd, kd, vd, meta, lse=lse, scale=0.07)
    torch.cuda.synchronize()
    p = plan["phases"][3]
    ref_o, ref_l = A.block_sparse_attention(q, k, v, p["kv_indices"], p["kv_counts"],
                                            global_tokens=plan["global_tokens"], scale=0.07)
    compare(out.cpu(), lse.cpu(), ref_o, ref_l, f"dtype {dtype} D {dim}")


def test_full_tables_equal_dense_sdpa(hip_device):
    """Dense gate: all-connection tables (plan.py:200-212) reproduce unmasked attention."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = T.full_attention_plan(oracle_plan("1024_t4k1"))
    q, k, v = _qkv(plan, heads=2, seed=5)
    qd, kd, vd = (x.to(hip_device) for x in (q, k, v))
    say("case full tables 1024")
    meta = device_paired(oracle_paired(plan, 0), hip_device)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=hip_device)
    out = paired_attention(qd, kd, vd, meta, lse=lse)
    torch.cuda.synchronize()
    qf, kf, vf = q.float(), k.float(), v.float()
    ref = F.scaled_dot_product_attention(qf, kf, vf)
    ref_lse = torch.logsumexp(torch.matmul(qf, kf.transpose(-1, -2).contiguous()) / D**0.5, -1)
    compare(out.cpu(), lse.cpu(), ref, ref_lse, "full tables vs SDPA")


def test_repeat_calls_bitwise_identical(hip_device):
    """The workspace queue counters reset themselves: back-to-back calls give identical bits."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t16k3")
    q, k, v = (x.to(hip_device) for x in _qkv(plan, heads=8, seed=9))
    meta = device_paired(oracle_paired(plan, 1), hip_device)
    say("case repeat calls")
    outs = [paired_attention(q, k, v, meta).clone() for _ in range(4)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


_QKV_2048: dict = {}


def _qkv_2048(plan, device):
    """Seed-2707 Q/K/V of a 2048 px config on the device, drawn once per module."""
    N = plan["total_tokens"]
    if N not in _QKV_2048:
        _QKV_2048.clear()
        _QKV_2048[N] = tuple(x.to(device) for x in _qkv(plan))
    return _QKV_2048[N]


@pytest.mark.parametrize("phase", range(4))
@pytest.mark.parametrize("name", ["2048_t16k3", "2048_t4k1"])
def test_paired_2048_full_output(hip_device, name, phase):
    """2048 px, 24 heads, every query row (global and ordinary), output and LSE, against the
    oracle's fp32 block formulation run on the device."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan(name)
    qd, kd, vd = _qkv_2048(plan, hip_device)
    say(f"case paired {name} phase {phase} full output")
    meta = device_paired(oracle_paired(plan, phase), hip_device)
    lse = torch.empty(qd.shape[:3], dtype=torch.float32, device=hip_device)
    out = paired_attention(qd, kd, vd, meta, global_strategy="triton", num_warps=8, lse=lse)
    torch.cuda.synchronize()
    ref_o, ref_l = reference(qd, kd, vd, plan, phase, device=hip_device)
    compare(out, lse, ref_o, ref_l, f"{name} phase {phase} all rows")


@pytest.mark.parametrize("phase", range(4))
def test_sparse_attention_2048_full_output(hip_device, phase):
    """The unpaired entry on the headline config: 64-query tables paired on the device, every
    row against the oracle's fp32 block formulation on the device."""
    from hilberta_amd.sparse_kernel import sparse_attention

    plan = oracle_plan("2048_t16k3")
    qd, kd, vd = _qkv_2048(plan, hip_device)
    p = plan["phases"][phase]
    say(f"case sparse_attention 2048_t16k3 phase {phase} full output")
    lse = torch.empty(qd.shape[:3], dtype=torch.float32, device=hip_device)
    out = sparse_attention(qd, kd, vd, torch.from_numpy(p["kv_indices"]).to(hip_device),
                           torch.from_numpy(p["kv_counts"]).to(hip_device),
                           global_tokens=plan["global_tokens"], global_strategy="triton", lse=lse)
    torch.cuda.synchronize()
    ref_o, ref_l = reference(qd, kd, vd, plan, phase, device=hip_device)
    compare(out, lse, ref_o, ref_l, f"sparse_attention 2048_t16k3 phase {phase} all rows")
