"""The C-ABI library loads without a GPU and exports every symbol include/hilberta_hip.h declares.

No compute entry point is called here except argument rejection paths that return before any
HIP call (HB_EINVAL), which exercise hb_last_error.
"""

import ctypes

from hilberta_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 10
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    assert lib.hb_version() == _lib.header_abi_version() == 4


def test_workspace_size_and_rejections():
    lib = _lib.load()
    ws = lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 512, 28, 64, 1, 1)
    assert ws > 64 * 1024
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 96, 512, 28, 64, 1, 1) == -1  # bad D
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 500, 28, 64, 1, 1) == -1  # bad G
    # argument checks return HB_EINVAL before touching the device
    strides = (ctypes.c_int64 * 12)(*([8] * 12))
    rc = lib.hb_paired_fwd(None, None, None, None, None, strides, 1, 1, 256, 128, 0, None, None, None,
                           1, 128, 64, 1, 1.0, None, 0, 0, None)
    assert rc == 1 and "null" in _lib.last_error()
    # quad tables: head_dim 128 and 64-key blocks only; N and G multiples of 256
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 512, 28, 64, 2, 1) > 64 * 1024
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 64, 512, 28, 64, 2, 1) == -1
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 512, 28, 128, 2, 1) == -1
    assert lib.hb_attention_workspace_bytes(1, 24, 16896 - 128, 128, 512, 28, 64, 2, 1) == -1
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 512, 28, 64, 3, 1) == -1
    rc = lib.hb_quad_rows(None, None, None, 4, 8, 64, None, None, None, 8, None, None)
    assert rc == 1 and "null" in _lib.last_error()
    # a lane's output row offset inside an item must fit 32 bits: the output token stride is bounded
    big = (ctypes.c_int64 * 12)(*([3072] * 11 + [(1 << 31) // 128]))
    rc = lib.hb_paired_fwd(16, 16, 16, 16, None, big, 1, 1, 256, 128, 0, 16, 16, 16, 1, 128, 64, 1,
                           1.0, 256, 1 << 20, 0, None)
    assert rc == 1 and "output token stride" in _lib.last_error()
    rc = lib.hb_hilbert_order(3, None, None)
    assert rc == 1 and "power of two" in _lib.last_error()
    assert lib.hb_plan_scratch_bytes(128, 64) == 256 * 256 * 4


def test_qk_prep_rejections():
    lib = _lib.load()
    def call(head_dim=128, normalize=1, eps=1e-6, text_tokens=512, weight=None, stride=3072):
        w = (ctypes.c_void_p * 2)(weight, None)
        return lib.hb_qk_prep(None, None, 0, stride, 0, stride, 1, 0, 1, text_tokens, 4608, 24,
                              head_dim, 0, normalize, w, eps, None, None, None, 0, 0, 3072, None)

    assert call(head_dim=64) == 1 and "head_dim" in _lib.last_error()
    assert call(text_tokens=5000) == 1 and "text_tokens" in _lib.last_error()
    assert call(normalize=1, eps=0.0) == 1
    assert call() == 1 and "null" in _lib.last_error()
    assert call(normalize=0, weight=16) == 1


def _global_chunks(batch, heads, tokens, global_tokens, width, head_dim=128):
    """Chunks per global query tile, read back from the workspace size of a paired launch.

    The workspace is 256 bytes of queue counters plus, per chunk of each 128-query global tile,
    the four waves' partial accumulators (head_dim/32 fragments x 16 x 64 fp32) and their
    (max, sum) rows (128 fp32); an unsplit tile needs no partials.
    """
    lib = _lib.load()
    ws = lib.hb_attention_workspace_bytes(batch, heads, tokens, head_dim, global_tokens, width,
                                          64, 1, 1)
    per_chunk = 4 * ((head_dim // 32) * 16 * 64 * 4 + 128 * 4)
    tiles = batch * heads * (global_tokens // 128)
    assert (ws - 256) % (tiles * per_chunk) == 0
    return max(1, (ws - 256) // (tiles * per_chunk))


def test_global_tile_split_plan():
    # FLUX 2048 px 16-tile K3 (264 key blocks, 128 paired rows of at most 28 entries): two chunks
    # of 132 blocks, about a workgroup's average work
    assert _global_chunks(1, 24, 16896, 512, 28) == 2
    # the same rows padded to twice the 64-query width (rows paired on the device without a host
    # sync) still split: one 264-block item per global tile would outlast the ordinary rows
    assert _global_chunks(1, 24, 16896, 512, 52) == 2
    # 2048 px 4-tile K1 (rows of 75 entries): a sweep shorter than four rows stays whole
    assert _global_chunks(1, 24, 16896, 512, 75) == 1
    # 1024 px (72 key blocks): chunks never fall below 64 steps' worth of target, so two of 36
    assert _global_chunks(1, 24, 4608, 512, 16) == 2
    assert _global_chunks(1, 24, 4608, 512, 27) == 2
    # a row as long as the whole key range leaves the global tiles unsplit
    assert _global_chunks(1, 24, 4608, 512, 72) == 1
    # 4096 px 16-tile K3 (1032 key blocks, width 75): two chunks of 516
    assert _global_chunks(1, 24, 66048, 512, 75) == 2
    # one head of it: thirteen chunks of 80 (merge_kernel's general path, past four chunks)
    assert _global_chunks(1, 1, 66048, 512, 75) == 13


def test_pair_rows_rejections():
    lib = _lib.load()
    buf = ctypes.c_void_p(16)  # never dereferenced: every call below fails its argument checks
    rc = lib.hb_pair_rows(buf, buf, 0, 4, 72, 64, buf, buf, buf, 8, None, None)
    assert rc == 1 and "rows must be positive" in _lib.last_error()
    rc = lib.hb_pair_rows(buf, buf, 4, 4, 16385, 64, buf, buf, buf, 8, None, None)
    assert rc == 1 and "total_blocks" in _lib.last_error()
    # quad rows keep 2048 key blocks
    rc = lib.hb_quad_rows(buf, buf, buf, 4, 8, 4096, buf, buf, buf, 8, None, None)
    assert rc == 1 and "total_blocks" in _lib.last_error()
    rc = lib.hb_pair_rows(buf, buf, 4, 4, 72, 96, buf, buf, buf, 8, None, None)
    assert rc == 1 and "key_block_size" in _lib.last_error()
    rc = lib.hb_pair_rows(None, buf, 4, 4, 72, 64, buf, buf, buf, 8, None, None)
    assert rc == 1 and "null" in _lib.last_error()


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """hb_paired_fwd_noalloc refuses shapes whose workspace exceeds its static scratch, before any
    HIP call; the limit is HB_NOALLOC_SCRATCH_BYTES (32 MiB)."""
    lib = _lib.load()
    limit = 32 << 20
    # a 2048-token global prefix at 2048 px: 16 global tiles per head, split in two
    need = lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 2048, 24, 64, 1, 1)
    assert need > limit
    buf = ctypes.c_void_p(4096)  # never dereferenced: the call fails its size check first
    strides = (ctypes.c_int64 * 12)(*([8] * 12))
    rc = lib.hb_paired_fwd_noalloc(buf, buf, buf, buf, None, strides, 1, 24, 16896, 128, 0, buf, buf,
                                   buf, 24, 2048, 64, 1, 1.0, 0, None)
    msg = _lib.last_error()
    assert rc == 1 and "scratch" in msg and str(need) in msg and str(limit) in msg
    # the shape checks shared with hb_paired_fwd come first
    rc = lib.hb_paired_fwd_noalloc(buf, buf, buf, buf, None, strides, 1, 24, 16896, 96, 0, buf, buf,
                                   buf, 24, 512, 64, 1, 1.0, 0, None)
    assert rc == 1 and "head_dim" in _lib.last_error()


def test_paired_ragged_shapes():
    """Paired launches take N and G in multiples of 64: ceil((N-G)/128) rows aligned to the end
    of the sequence and ceil(G/128) global tiles, the last of which overhangs G when G is an odd
    multiple of 64; the split partials in the workspace count that tile whole."""
    lib = _lib.load()
    per_chunk = 4 * (4 * 16 * 64 * 4 + 128 * 4)  # four waves' fragments and (max, sum) rows
    for G, tiles in ((512, 4), (576, 5), (64, 1)):
        N = 16896 + (G - 512)
        ws = lib.hb_attention_workspace_bytes(1, 24, N, 128, G, 28, 64, 1, 1)
        assert (ws - 256) == 24 * tiles * 2 * per_chunk, (G, ws)  # two chunks of 132 blocks
    assert lib.hb_attention_workspace_bytes(1, 24, 16384, 128, 0, 28, 64, 1, 1) == 256
    # N - G an odd multiple of 64 is accepted; N or G off the 64 grid is not
    assert lib.hb_attention_workspace_bytes(1, 24, 16896 - 64, 128, 512, 28, 64, 1, 1) > 256
    assert lib.hb_attention_workspace_bytes(1, 24, 16896 - 32, 128, 512, 28, 64, 1, 1) == -1
    assert lib.hb_attention_workspace_bytes(1, 24, 16896, 128, 544, 28, 64, 1, 1) == -1
    # quad tables keep multiples of 256
    assert lib.hb_attention_workspace_bytes(1, 24, 16896 - 128, 128, 512, 28, 64, 2, 1) == -1
    # hb_pair_rows takes odd row counts (paired from the end); only the count's sign is checked
    buf = ctypes.c_void_p(16)
    rc = lib.hb_pair_rows(buf, buf, -3, 4, 72, 64, buf, buf, buf, 8, None, None)
    assert rc == 1 and "rows must be positive" in _lib.last_error()


def test_plain_c_host_builds_a_paired_phase(tmp_path):
    """A plain C program (tests/c/host_plan.c, gcc -std=c99, the header as is) links the library,
    builds one phase of a bridge_k plan with the host entry points and pairs it: its output equals
    the oracle's bridge_k_plan + pair_metadata, without a GPU."""
    import shutil
    import subprocess
    from pathlib import Path

    import pytest

    from oracle import topology as T

    if shutil.which("gcc") is None:
        pytest.skip("gcc is not installed")
    root = Path(__file__).resolve().parents[1]
    exe = tmp_path / "host_plan"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-O2", f"-I{root / 'include'}",
                    str(root / "tests" / "c" / "host_plan.c"), f"-L{root / 'hilberta_amd'}",
                    "-lhilberta_hip", f"-Wl,-rpath,{root / 'hilberta_amd'}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    for grid, tiles, k, phase, kb in ((64, 16, 3, 1, 64), (128, 4, 2, 3, 128), (128, 16, 3, 2, 64)):
        out = subprocess.run([str(exe), str(grid), str(tiles), str(k), str(phase), str(kb)],
                             check=True, capture_output=True, text=True).stdout.splitlines()
        plan = T.bridge_k_plan(tiles, k, False, grid_size=grid)
        p = plan["phases"][phase]
        ref = T.pair_metadata(p["kv_indices"], p["kv_counts"], tokens=plan["total_tokens"],
                              global_tokens=plan["global_tokens"], key_block_size=kb)
        assert out[0] == "shared 0"
        rows, width = ref["kv_indices"].shape
        assert out[1] == f"rows {rows} width {width}"
        for r, line in enumerate(out[2:]):
            count, _, entries = line.partition(":")
            pairs = [tuple(map(int, e.split("/"))) for e in entries.split()]
            assert int(count) == ref["kv_counts"][r] == len(pairs)
            assert [b for b, _ in pairs] == ref["kv_indices"][r, :len(pairs)].tolist()
            assert [f for _, f in pairs] == ref["kv_flags"][r, :len(pairs)].tolist()
        assert len(out) == 2 + rows
