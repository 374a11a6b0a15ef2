"""The torch custom ops (hilberta_amd/ops.py) on the CPU: schemas, fake implementations under
FakeTensorMode (shapes only, no kernel), no CPU kernel for the attention and gather ops (pair_rows,
plan setup, has one), and the entry points' routing through the ops.  Real launches and torch.library.opcheck run in tests/test_gpu_ops.py."""

from unittest.mock import patch

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import hilberta_amd  # noqa: F401  (registers the ops)

OPS = torch.ops.hilberta_hip


def test_schemas_declare_the_written_outputs():
    paired = str(OPS.paired_fwd.default._schema)
    sparse = str(OPS.sparse_fwd.default._schema)
    for schema in (paired, sparse):
        assert "Tensor(a3!) out" in schema and "Tensor(a4!)? lse" in schema and schema.endswith("-> ()")
        assert "Tensor q," in schema and "Tensor kv_indices" in schema  # inputs are read only
    assert str(OPS.gather_rows.default._schema).endswith("-> Tensor")
    assert str(OPS.pair_rows.default._schema).endswith("-> (Tensor, Tensor, Tensor)")


def test_fake_implementations_propagate_shapes():
    with FakeTensorMode():
        x = torch.empty(2, 4096, 64, dtype=torch.bfloat16, device="cuda")
        order = torch.empty(4096, dtype=torch.int64, device="cuda")
        y = OPS.gather_rows(x, 1, order)
        assert y.shape == (2, 4096, 64) and y.dtype == torch.bfloat16 and y.device.type == "cuda"
        ids = torch.empty(64, 20, dtype=torch.int32, device="cuda")
        counts = torch.empty(64, dtype=torch.int32, device="cuda")
        pid, pfl, pct = OPS.pair_rows(ids, counts, 72, 64, 40)
        assert pid.shape == pfl.shape == (32, 40) and pct.shape == (32,) and pid.dtype == torch.int32
        q = torch.empty(1, 2, 4608, 128, dtype=torch.bfloat16, device="cuda")
        out = torch.empty_like(q)
        lse = torch.empty(1, 2, 4608, dtype=torch.float32, device="cuda")
        assert OPS.paired_fwd(q, q, q, out, lse, pid, pfl, pct, 512, 64, 0.1, True, 0) is None
        assert OPS.sparse_fwd(q, q, q, out, None, ids, counts, 512, 0.1, True, 0) is None


def test_no_cpu_kernel():
    x = torch.zeros(4, 3)
    with pytest.raises(NotImplementedError):
        OPS.gather_rows(x, 0, torch.arange(4))


def test_pair_rows_op_on_cpu_tensors():
    """pair_rows is plan setup: on CPU tensors it runs the host builder and equals the oracle's
    pair_metadata (reference paired_metadata.py:26-51)."""
    from oracle import topology as T

    plan = T.bridge_k_plan(16, 3, False, grid_size=64)
    p = plan["phases"][1]
    ref = T.pair_metadata(p["kv_indices"], p["kv_counts"], tokens=plan["total_tokens"],
                          global_tokens=plan["global_tokens"], key_block_size=128)
    width = ref["kv_indices"].shape[1]
    ids, flags, counts = OPS.pair_rows(torch.from_numpy(p["kv_indices"]),
                                       torch.from_numpy(p["kv_counts"]),
                                       plan["total_tokens"] // 64, 128, width)
    assert ids.device.type == "cpu"
    assert ids.numpy().tolist() == ref["kv_indices"].tolist()
    assert flags.numpy().tolist() == ref["kv_flags"].tolist()
    assert counts.numpy().tolist() == ref["kv_counts"].tolist()
    torch.library.opcheck(OPS.pair_rows.default, (torch.from_numpy(p["kv_indices"]),
                                                  torch.from_numpy(p["kv_counts"]),
                                                  plan["total_tokens"] // 64, 128, width))


def test_entry_points_call_the_ops():
    """paired_attention / sparse_attention / index_select_rows reach torch.ops.hilberta_hip.*
    after their host checks (the ops themselves are patched out: no GPU here)."""
    from types import SimpleNamespace

    from hilberta_amd import layout, ops, paired_kernel, sparse_kernel
    from tests.test_contract import NATIVE, SHAPE, HostView

    q, k, v = (HostView(SHAPE, NATIVE, address=a) for a in (1 << 20, 2 << 20, 3 << 20))
    ids, flags = (HostView((3, 5), dtype=torch.int32, address=a) for a in (4 << 20, 5 << 20))
    counts = HostView((3,), dtype=torch.int32, address=6 << 20)
    meta = SimpleNamespace(tokens=512, global_tokens=128, key_block_size=64, kv_indices=ids,
                           kv_flags=flags, kv_counts=counts)
    out = HostView(SHAPE, NATIVE, address=7 << 20)
    with patch.object(ops, "paired_fwd") as op:
        assert paired_kernel.paired_attention(q, k, v, meta, out=out) is out
    assert op.call_count == 1
    assert op.call_args.args[:8] == (q, k, v, out, None, ids, flags, counts)
    assert op.call_args.args[8:] == (128, 64, pytest.approx(128**-0.5 * sparse_kernel.LOG2E), True,
                                     paired_kernel.NUM_GROUPS)
    uids = HostView((6, 5), dtype=torch.int32, address=4 << 20)
    ucounts = HostView((6,), dtype=torch.int32, address=5 << 20)
    with patch.object(ops, "sparse_fwd") as op:
        sparse_kernel.sparse_attention(q, k, v, uids, ucounts, global_tokens=128, out=out)
    assert op.call_count == 1 and op.call_args.args[5:8] == (uids, ucounts, 128)
    with patch.object(ops, "gather_rows") as op, patch.object(layout._lib, "require_gpu"):
        layout.index_select_rows(torch.zeros(1, 8, 4), 1, torch.arange(8))
    assert op.call_count == 1 and op.call_args.args[1] == 1
