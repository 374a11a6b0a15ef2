"""The torch custom ops on the GPU: torch.library.opcheck (schema and declared mutations, fake
implementation against the real one, tracing through AOT dispatch) for each operator, and one
call through the operator bitwise equal to the same launch made directly through the C ABI."""

import ctypes

import numpy as np
import pytest
import torch

import hilberta_amd  # noqa: F401  (registers the ops)
from oracle import attention as A
from tests.helpers import device_paired, oracle_paired, oracle_plan, say

pytestmark = pytest.mark.gpu

OPS = torch.ops.hilberta_hip
D = 128


@pytest.fixture(scope="module")
def case(hip_device):
    plan = oracle_plan("1024_t16k3")
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 2, plan["total_tokens"], D, seed=29))
    meta = device_paired(oracle_paired(plan, 1), hip_device)
    p = plan["phases"][1]
    ids = torch.from_numpy(p["kv_indices"]).to(hip_device)
    counts = torch.from_numpy(p["kv_counts"]).to(hip_device)
    return plan, q, k, v, meta, ids, counts


def _paired_args(case, out, lse):
    plan, q, k, v, meta, _, _ = case
    return (q, k, v, out, lse, meta.kv_indices, meta.kv_flags, meta.kv_counts, plan["global_tokens"],
            64, D**-0.5 * 1.4426950408889634, True, 0)


def test_opcheck_paired_fwd(case):
    q = case[1]
    say("case opcheck paired_fwd")
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    torch.library.opcheck(OPS.paired_fwd.default, _paired_args(case, torch.empty_like(q), lse))
    torch.library.opcheck(OPS.paired_fwd.default, _paired_args(case, torch.empty_like(q), None))


def test_opcheck_sparse_fwd(case):
    plan, q, k, v, _, ids, counts = case
    say("case opcheck sparse_fwd")
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    torch.library.opcheck(OPS.sparse_fwd.default, (q, k, v, torch.empty_like(q), lse, ids, counts,
                                                   plan["global_tokens"], 0.1, True, 0))


def test_opcheck_gather_and_pair_rows(case):
    _, q, _, _, _, ids, counts = case
    say("case opcheck gather_rows / pair_rows")
    x = torch.randn(2, 4096, 64, device=q.device).to(torch.bfloat16)
    order = torch.randperm(4096, device=q.device)
    torch.library.opcheck(OPS.gather_rows.default, (x, 1, order))
    torch.library.opcheck(OPS.pair_rows.default, (ids, counts, q.shape[2] // 64, 64,
                                                  min(2 * ids.shape[1], q.shape[2] // 64)))


def test_op_call_equals_direct_c_abi_launch(case):
    from hilberta_amd import _lib
    from hilberta_amd._workspace import attention_workspace

    plan, q, k, v, meta, _, _ = case
    G, N = plan["global_tokens"], q.shape[2]
    say("case op vs direct hb_paired_fwd")
    out_op, out_c = torch.empty_like(q), torch.empty_like(q)
    lse_op = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    lse_c = torch.empty_like(lse_op)
    OPS.paired_fwd(*_paired_args(case, out_op, lse_op))
    width = meta.kv_indices.shape[1]
    ws = attention_workspace(q.device, 1, 2, N, D, G, width, 64, paired=1, all_queries=1)
    strides = (ctypes.c_int64 * 12)(*[s for x in (q, k, v, out_c) for s in x.stride()[:3]])
    rc = _lib.load().hb_paired_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out_c.data_ptr(), lse_c.data_ptr(), strides, 1, 2,
        N, D, 0, meta.kv_indices.data_ptr(), meta.kv_flags.data_ptr(), meta.kv_counts.data_ptr(),
        width, G, 64, 1, D**-0.5 * 1.4426950408889634, ws.data_ptr(), ws.numel(), 0,
        _lib.stream_ptr(q.device))
    _lib.check(rc, "hb_paired_fwd")
    torch.cuda.synchronize()
    assert torch.equal(out_op, out_c) and torch.equal(lse_op, lse_c)
    # and through the Python entry point, which calls the operator
    from hilberta_amd.paired_kernel import paired_attention

    lse_py = torch.empty_like(lse_op)
    out_py = paired_attention(q, k, v, meta, lse=lse_py)
    assert torch.equal(out_py, out_c) and torch.equal(lse_py, lse_c)
    # gather: bit for bit with index_select
    x = torch.randn(1, 4096, 3072, device=q.device).to(torch.bfloat16)
    order = torch.from_numpy(np.random.default_rng(1).permutation(4096)).to(q.device)
    assert torch.equal(OPS.gather_rows(x, 1, order), x.index_select(1, order))
