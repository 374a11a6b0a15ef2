"""paired_attention captured in a HIP graph (torch.cuda.CUDAGraph) replays bitwise like eager calls.

The launch path allocates nothing beyond a per-(device, stream) workspace that is zero-filled by a
fill kernel when first made, and the persistent kernel's work-queue counters are left at zero by
the last workgroup of every launch, so a captured step can be replayed any number of times.  The
graph is replayed several times with eager work and synchronisations between replays, and every
replay is checked against the eager result; a replay after an in-place update of Q must see the
new values.
"""

import pytest
import torch

from tests.helpers import device_paired, oracle_paired, oracle_plan, say
from oracle import attention as A

pytestmark = pytest.mark.gpu


def test_paired_step_graph_replays_match_eager(hip_device):
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t16k3")
    N = plan["total_tokens"]
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 8, N, 128, seed=31))
    q2 = A.seeded_qkv(1, 8, N, 128, seed=32)[0].to(hip_device)
    metas = [device_paired(oracle_paired(plan, p), hip_device) for p in range(4)]

    def step(outs, lses):
        for m, o, l in zip(metas, outs, lses):
            paired_attention(q, k, v, m, out=o, lse=l)

    def buffers():
        return ([torch.empty_like(q) for _ in metas],
                [torch.empty(1, 8, N, dtype=torch.float32, device=hip_device) for _ in metas])

    say("case graph: eager reference for two Q inputs")
    q_first = q.clone()
    eager1, eager1_lse = buffers()
    step(eager1, eager1_lse)
    q.copy_(q2)
    eager2, eager2_lse = buffers()
    step(eager2, eager2_lse)
    q.copy_(q_first)
    torch.cuda.synchronize()

    say("case graph: warm-up and capture of the 4-phase step")
    outs, lses = buffers()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(outs, lses)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(outs, lses)
    torch.cuda.synchronize()

    for rep in range(3):
        say(f"case graph: replay {rep}")
        for o, l in zip(outs, lses):
            o.zero_()
            l.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for p in range(4):
            assert torch.equal(outs[p], eager1[p]), f"replay {rep} phase {p} output"
            assert torch.equal(lses[p], eager1_lse[p]), f"replay {rep} phase {p} lse"
        # eager work on the same stream between replays
        x = paired_attention(q, k, v, metas[rep])
        torch.cuda.synchronize()
        assert torch.equal(x, eager1[rep])

    say("case graph: replay after an in-place update of Q")
    q.copy_(q2)
    graph.replay()
    torch.cuda.synchronize()
    for p in range(4):
        assert torch.equal(outs[p], eager2[p]), f"updated Q, phase {p} output"
        assert torch.equal(lses[p], eager2_lse[p]), f"updated Q, phase {p} lse"


def test_two_graphs_on_one_capture_stream_replay_concurrently(hip_device):
    """Graphs captured one after another on torch's shared capture stream get workspaces of
    their own (each from its graph's private pool, none from the eager cache), so replaying them
    at the same time on two streams gives each its eager result."""
    from hilberta_amd import _workspace
    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("2048_t16k3")
    N = plan["total_tokens"]
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 6, N, 128, seed=33))
    metas = [device_paired(oracle_paired(plan, p), hip_device) for p in range(2)]
    eager = [paired_attention(q, k, v, m) for m in metas]
    outs = [torch.empty_like(q) for _ in metas]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for m, o in zip(metas, outs):
            paired_attention(q, k, v, m, out=o)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    say("case two graphs captured on the shared capture stream")
    before = set(_workspace._CACHE)
    graphs = [torch.cuda.CUDAGraph() for _ in metas]
    for g, m, o in zip(graphs, metas, outs):
        with torch.cuda.graph(g):
            paired_attention(q, k, v, m, out=o)
    torch.cuda.synchronize()
    assert set(_workspace._CACHE) == before  # captured launches leave the eager cache alone
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(4):
        say(f"case concurrent replay {rep}")
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        for g, s in zip(graphs, streams):
            with torch.cuda.stream(s):
                g.replay()
        torch.cuda.synchronize()
        for p in range(2):
            assert torch.equal(outs[p], eager[p]), f"replay {rep} graph {p}"


def test_captures_hold_no_memory_after_their_graphs(hip_device):
    """A captured launch's workspace lives in its graph's private pool: capturing and dropping
    graphs repeatedly leaves the allocated memory where it started."""
    import gc

    from hilberta_amd.paired_kernel import paired_attention

    plan = oracle_plan("1024_t16k3")
    N = plan["total_tokens"]
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 4, N, 128, seed=33))
    meta = device_paired(oracle_paired(plan, 0), hip_device)
    out = torch.empty_like(q)
    ref = paired_attention(q, k, v, meta)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()

    def capture_once():
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            paired_attention(q, k, v, meta, out=out)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            paired_attention(q, k, v, meta, out=out)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        del g
        gc.collect()
        torch.cuda.synchronize()

    say("case graph: repeated capture and release")
    capture_once()
    before = torch.cuda.memory_allocated(hip_device)
    for _ in range(4):
        capture_once()
    assert torch.cuda.memory_allocated(hip_device) == before


def test_sparse_attention_ragged_graph_replays_match_eager(hip_device):
    """sparse_attention on a table that pairs only with overhanging halves (an odd row count and
    a global prefix that is an odd multiple of 64) captured in a HIP graph: the device pairing
    launch and the paired forward replay bitwise like the eager call, with eager work between
    replays."""
    import numpy as np

    from hilberta_amd.sparse_kernel import sparse_attention

    G, rows = 576, 71
    N = G + 64 * rows
    T_ = N // 64
    rng = np.random.default_rng(41)
    width = G // 64 + 6
    ids = np.zeros((rows, width), np.int32)
    counts = np.zeros(rows, np.int32)
    for r in range(rows):
        extra = rng.choice(np.arange(G // 64, T_), size=rng.integers(1, 7), replace=False)
        row = np.concatenate([np.arange(G // 64), np.sort(extra)]).astype(np.int32)
        ids[r, :len(row)] = row
        counts[r] = len(row)
    idd, cnd = torch.from_numpy(ids).to(hip_device), torch.from_numpy(counts).to(hip_device)
    q, k, v = (x.to(hip_device) for x in A.seeded_qkv(1, 4, N, 128, seed=43))
    eager_lse = torch.empty(1, 4, N, dtype=torch.float32, device=hip_device)
    eager = sparse_attention(q, k, v, idd, cnd, global_tokens=G, lse=eager_lse)
    out = torch.empty_like(q)
    lse = torch.empty_like(eager_lse)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sparse_attention(q, k, v, idd, cnd, global_tokens=G, out=out, lse=lse)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    say("case graph: sparse_attention on a ragged table")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sparse_attention(q, k, v, idd, cnd, global_tokens=G, out=out, lse=lse)
    torch.cuda.synchronize()
    for rep in range(3):
        say(f"case graph ragged: replay {rep}")
        out.zero_()
        lse.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} output"
        assert torch.equal(lse, eager_lse), f"replay {rep} lse"
        x = sparse_attention(q, k, v, idd, cnd, global_tokens=G)
        torch.cuda.synchronize()
        assert torch.equal(x, eager)
