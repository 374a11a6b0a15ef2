"""GPU edge cases of the attention path: table padding, the C ABI's all_queries=0 mode, 4096 px
(sampled rows, and every row of all four phases), D = 64 and the adapter's BNHD storage at
2048 px (every row; the D = 64 kernel runs three workgroups per CU there), B=2 with BNHD views and
128-key tables at 2048 px, and the permutation at 4096 px sizes.

References are the fp32 oracle formulations in oracle/attention.py (block form on sampled query
tiles, computed on the device in fp32), the kernel's own all_queries=1 output (bitwise), and
torch's index_select (bitwise).
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as A
from tests.helpers import compare, device_paired, oracle_paired, oracle_plan, say

pytestmark = pytest.mark.gpu

D = 128


def _sampled_rows_check(out, lse, qd, kd, vd, plan, phase, rows, what, key_block_size=64):
    """Ordinary paired rows `rows` (64-query blocks) against the block formulation in fp32."""
    G = plan["global_tokens"]
    p = plan["phases"][phase]
    qf, kf, vf = qd.float(), kd.float(), vd.float()
    for row in rows:
        q0 = G + 64 * row
        ids = p["kv_indices"][row, : p["kv_counts"][row]]
        cols = torch.from_numpy((ids[:, None] * 64 + np.arange(64)).reshape(-1)).to(qd.device)
        s = torch.matmul(qf[:, :, q0 : q0 + 64], kf[:, :, cols].transpose(-1, -2).contiguous())
        s = s * D**-0.5
        rl = torch.logsumexp(s, -1)
        ro = torch.matmul(torch.softmax(s, -1), vf[:, :, cols])
        compare(out[:, :, q0 : q0 + 64], None if lse is None else lse[:, :, q0 : q0 + 64], ro, rl,
                f"{what} row {row}")


def test_table_padding_is_ignored(hip_device):
    """Entries past a row's count may hold anything (sparse_kernel.py:140-152): same bits."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t16k3")
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 4, plan["total_tokens"], D, seed=3))
    meta_np = oracle_paired(plan, 2)
    clean = device_paired(meta_np, hip_device)
    ids = meta_np["kv_indices"].copy()
    flags = meta_np["kv_flags"].copy()
    counts = meta_np["kv_counts"]
    width = ids.shape[1]
    rng = np.random.default_rng(1)
    pad = np.arange(width)[None, :] >= counts[:, None]
    assert pad.any(), "the phase needs ragged rows for this test"
    ids[pad] = rng.integers(-(1 << 30), 1 << 30, size=int(pad.sum()))
    flags[pad] = rng.integers(0, 16, size=int(pad.sum()))
    dirty = device_paired(dict(meta_np, kv_indices=ids, kv_flags=flags), hip_device)
    say("case padding garbage 1024_t16k3 phase 2")
    a = paired_attention(q, k, v, clean)
    b = paired_attention(q, k, v, dirty)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_c_abi_all_queries_zero_keeps_global_rows(hip_device):
    """hb_paired_fwd(all_queries=0) computes only the ordinary rows (the reference's ALL_QUERIES=0
    launch under global_strategy="flash", paired_kernel.py:173-178) and leaves the global rows."""
    from hilberta_amd import _lib
    from hilberta_amd._workspace import attention_workspace
    from hilberta_amd.paired_kernel import paired_attention
    from hilberta_amd.sparse_kernel import LOG2E, _strides

    plan = oracle_plan("1024_t4k1")
    N, G = plan["total_tokens"], plan["global_tokens"]
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 6, N, D, seed=4))
    meta = device_paired(oracle_paired(plan, 1), hip_device)
    full = paired_attention(q, k, v, meta)
    out = torch.full_like(q, 7.0)
    lib = _lib.load()
    width = meta.kv_indices.shape[1]
    ws = attention_workspace(q.device, 1, 6, N, D, G, width, 64, paired=1, all_queries=0)
    strides = (ctypes.c_int64 * 12)(*_strides(q, k, v, out))
    say("case all_queries=0 via the C ABI")
    rc = lib.hb_paired_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), None, strides,
                           1, 6, N, D, 0, meta.kv_indices.data_ptr(), meta.kv_flags.data_ptr(),
                           meta.kv_counts.data_ptr(), width, G, 64, 0, D**-0.5 * LOG2E,
                           ws.data_ptr(), ws.numel(), 0, _lib.stream_ptr(q.device))
    _lib.check(rc, "hb_paired_fwd")
    torch.cuda.synchronize()
    assert bool((out[:, :, :G] == 7.0).all()), "global rows were written"
    assert torch.equal(out[:, :, G:], full[:, :, G:])


def test_paired_4096_sampled_rows(hip_device):
    """4096 px 16-tile K3 (the largest config): global rows on 2 heads and 12 sampled rows."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("4096_t16k3")
    N, G = plan["total_tokens"], plan["global_tokens"]
    heads = 8
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, heads, N, D, seed=6))
    phase = 1
    meta = device_paired(oracle_paired(plan, phase), hip_device)
    lse = torch.empty(1, heads, N, dtype=torch.float32, device=hip_device)
    say("case paired 4096_t16k3 phase 1")
    out = paired_attention(q, k, v, meta, lse=lse)
    torch.cuda.synchronize()
    qf, kf, vf = q[:, :2].float(), k[:, :2].float(), v[:, :2].float()
    s = torch.matmul(qf[:, :, :G], kf.transpose(-1, -2).contiguous()) * D**-0.5
    compare(out[:, :2, :G], lse[:, :2, :G], torch.matmul(torch.softmax(s, -1), vf),
            torch.logsumexp(s, -1), "4096 global rows")
    del s
    nq = len(plan["phases"][phase]["kv_counts"])
    rows = sorted(set(np.random.default_rng(2).choice(nq, 12, replace=False).tolist()) | {0, nq - 1})
    _sampled_rows_check(out, lse, q, k, v, plan, phase, rows, "4096")


def test_paired_4096_one_head_many_chunks(hip_device):
    """One head at 4096 px: the planner splits each global tile into 13 chunks (more than the
    merge kernel's four-chunk fast path takes, tests/test_capi.py), so the general merge runs;
    global rows against fp32 attention over all keys, and sampled ordinary rows."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("4096_t16k3")
    N, G = plan["total_tokens"], plan["global_tokens"]
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 1, N, D, seed=12))
    phase = 3
    meta = device_paired(oracle_paired(plan, phase), hip_device)
    lse = torch.empty(1, 1, N, dtype=torch.float32, device=hip_device)
    say("case paired 4096_t16k3 one head, global tiles in 13 chunks")
    out = paired_attention(q, k, v, meta, lse=lse)
    torch.cuda.synchronize()
    qf, kf, vf = q.float(), k.float(), v.float()
    s = torch.matmul(qf[:, :, :G], kf.transpose(-1, -2).contiguous()) * D**-0.5
    compare(out[:, :, :G], lse[:, :, :G], torch.matmul(torch.softmax(s, -1), vf),
            torch.logsumexp(s, -1), "4096 one head global rows")
    nq = len(plan["phases"][phase]["kv_counts"])
    rows = sorted(set(np.random.default_rng(5).choice(nq, 8, replace=False).tolist()) | {0, nq - 1})
    _sampled_rows_check(out, lse, q, k, v, plan, phase, rows, "4096 one head")


_QKV_4096: dict = {}


def _block_reference_all_heads(qd, kd, vd, plan, phase):
    """oracle.attention.block_sparse_attention's block formulation in fp32 on the device, with
    each 64-query row computed for every head in one batched product (the oracle loops over
    heads, which at 4096 px means 24k small launches per phase)."""
    G = plan["global_tokens"]
    p = plan["phases"][phase]
    scale = qd.shape[-1] ** -0.5
    qf, kf, vf = qd.float(), kd.float(), vd.float()
    ref_o = torch.empty_like(qf)
    ref_l = torch.empty(qf.shape[:3], dtype=torch.float32, device=qf.device)
    for h0 in range(0, qf.shape[1], 6):
        hs = slice(h0, h0 + 6)
        s = torch.matmul(qf[:, hs, :G], kf[:, hs].transpose(-1, -2).contiguous()) * scale
        ref_l[:, hs, :G] = torch.logsumexp(s, -1)
        ref_o[:, hs, :G] = torch.matmul(torch.softmax(s, -1), vf[:, hs])
        del s
    ids_all = torch.from_numpy(p["kv_indices"].astype(np.int64)).to(qd.device)
    for row, count in enumerate(p["kv_counts"].tolist()):
        q0 = G + 64 * row
        cols = (ids_all[row, :count, None] * 64 + torch.arange(64, device=qd.device)).reshape(-1)
        s = torch.matmul(qf[:, :, q0 : q0 + 64], kf[:, :, cols].transpose(-1, -2).contiguous())
        s = s * scale
        ref_l[:, :, q0 : q0 + 64] = torch.logsumexp(s, -1)
        ref_o[:, :, q0 : q0 + 64] = torch.matmul(torch.softmax(s, -1), vf[:, :, cols])
    return ref_o, ref_l


@pytest.mark.parametrize("phase", range(4))
def test_paired_4096_full_output(hip_device, phase):
    """4096 px 16-tile K3 (N = 66048, the largest config), 24 heads: every query row of the
    phase, output and LSE, against the block formulation in fp32 on the device."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("4096_t16k3")
    N = plan["total_tokens"]
    if N not in _QKV_4096:
        _QKV_4096.clear()
        _QKV_4096[N] = tuple(x.to(hip_device) for x in A.seeded_qkv(1, 24, N, D, seed=2707))
    q, k, v = _QKV_4096[N]
    say(f"case paired 4096_t16k3 phase {phase} full output")
    meta = device_paired(oracle_paired(plan, phase), hip_device)
    lse = torch.empty(1, 24, N, dtype=torch.float32, device=hip_device)
    out = paired_attention(q, k, v, meta, global_strategy="triton", lse=lse)
    torch.cuda.synchronize()
    ref_o, ref_l = _block_reference_all_heads(q, k, v, plan, phase)
    compare(out, lse, ref_o, ref_l, f"4096_t16k3 phase {phase} all rows")


def test_paired_2048_adapter_layout_full_output(hip_device):
    """The adapter's storage (flux_adapter.py:280-326): Q/K/V projected as [B, N, H, D] and
    viewed as [B, H, N, D] (strides N*H*D, D, H*D, 1), 2048 px 16-tile K3, 24 heads: every row of
    one phase, output (in the same storage order) and LSE, against the block formulation."""
    from hilberta_amd.paired_kernel import paired_attention

    _QKV_4096.clear()
    plan = oracle_plan("2048_t16k3")
    N = plan["total_tokens"]
    q, k, v = A.seeded_qkv(1, 24, N, D, seed=13)
    qd, kd, vd = (x.transpose(1, 2).contiguous().to(hip_device).transpose(1, 2) for x in (q, k, v))
    assert qd.stride() == (N * 24 * D, D, 24 * D, 1)
    say("case paired 2048_t16k3 BNHD views phase 1 full output")
    meta = device_paired(oracle_paired(plan, 1), hip_device)
    lse = torch.empty(1, 24, N, dtype=torch.float32, device=hip_device)
    out = paired_attention(qd, kd, vd, meta, lse=lse)
    torch.cuda.synchronize()
    assert out.stride() == qd.stride()
    ref_o, ref_l = _block_reference_all_heads(qd, kd, vd, plan, 1)
    compare(out, lse, ref_o, ref_l, "2048_t16k3 BNHD views all rows")


@pytest.mark.parametrize("f16", [False, True])
def test_paired_2048_head_dim_64_full_output(hip_device, f16):
    """D = 64 at 2048 px 16-tile K3, 24 heads (3360 items: the D = 64 kernel then runs three
    workgroups per CU): every query row, output and LSE, against the block formulation."""
    from hilberta_amd.paired_kernel import paired_attention

    _QKV_4096.clear()
    plan = oracle_plan("2048_t16k3")
    N = plan["total_tokens"]
    dtype = torch.float16 if f16 else torch.bfloat16
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 24, N, 64, seed=11, dtype=dtype))
    say(f"case paired 2048_t16k3 D=64 {'fp16' if f16 else 'bf16'} phase 2 full output")
    meta = device_paired(oracle_paired(plan, 2), hip_device)
    lse = torch.empty(1, 24, N, dtype=torch.float32, device=hip_device)
    out = paired_attention(q, k, v, meta, lse=lse)
    torch.cuda.synchronize()
    ref_o, ref_l = _block_reference_all_heads(q, k, v, plan, 2)
    compare(out, lse, ref_o, ref_l, f"2048_t16k3 D=64 {'fp16' if f16 else 'bf16'} all rows")


def test_paired_2048_batch2_bnhd_key_block_128(hip_device):
    """B=2, the adapter's BNHD storage viewed as BHND, 128-key paired tables, at 2048 px."""
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("2048_t16k3")
    N = plan["total_tokens"]
    heads = 6
    q, k, v = A.seeded_qkv(2, heads, N, D, seed=8)
    to_bnhd = lambda x: x.transpose(1, 2).contiguous().to(hip_device).transpose(1, 2)  # noqa: E731
    qd, kd, vd = to_bnhd(q), to_bnhd(k), to_bnhd(v)
    meta = device_paired(oracle_paired(plan, 3, key_block_size=128), hip_device)
    lse = torch.empty(2, heads, N, dtype=torch.float32, device=hip_device)
    say("case paired 2048 B=2 BNHD KB128 phase 3")
    out = paired_attention(qd, kd, vd, meta, lse=lse)
    torch.cuda.synchronize()
    nq = len(plan["phases"][3]["kv_counts"])
    rows = sorted(set(np.random.default_rng(3).choice(nq, 16, replace=False).tolist()) | {0, nq - 1})
    _sampled_rows_check(out, lse, qd, kd, vd, plan, 3, rows, "2048 B=2 KB128")


@pytest.mark.parametrize("shape", [(1, 100_000_000, 3), (1500, 1_000_000, 3)])
def test_permutation_byte_rows_long_walks(hip_device, shape):
    """3-byte rows move one byte per thread: 3e8 bytes take the grid-stride loop of the 32-bit
    walk, 4.5e9 bytes the 64-bit walk; both bit-exact against torch's index_select."""
    from hilberta_amd.layout import index_select_rows

    gen = torch.Generator(hip_device).manual_seed(13)
    x = torch.randint(0, 256, shape, dtype=torch.uint8, device=hip_device, generator=gen)
    index = torch.randperm(shape[1], device=hip_device, generator=gen)
    say(f"case byte-row permutation {shape}")
    out = index_select_rows(x, 1, index)
    assert torch.equal(out, x.index_select(1, index))
    del out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("shape,dim", [((1, 65536, 64), 1), ((1, 66048, 24, 128), 1)])
def test_permutation_4096_sizes(hip_device, shape, dim):
    """4096 px latents and BNHD projections: gather and its inverse are bit-exact."""
    from hilberta_amd.layout import index_select_rows

    gen = torch.Generator("cpu").manual_seed(12)
    x = torch.randn(shape, generator=gen).to(torch.bfloat16).to(hip_device)
    index = torch.randperm(shape[dim], generator=gen).to(hip_device)
    say(f"case permutation {shape}")
    out = index_select_rows(x, dim, index)
    assert torch.equal(out, x.index_select(dim, index))
    inv = torch.empty_like(index)
    inv[index] = torch.arange(len(index), device=hip_device)
    assert torch.equal(index_select_rows(out, dim, inv), x)
