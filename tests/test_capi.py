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
    assert lib.hb_version() == 1


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
