"""ctypes binding of libhilberta_hip.so (declarations in include/hilberta_hip.h).

There is no fallback: if the library is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libhilberta_hip.so"
HEADER = _PKG.parent / "include" / "hilberta_hip.h"

HB_EINVAL = 1

_c_int, _c_i64, _c_f32, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/hilberta_hip.h
SIGNATURES = {
    "hb_last_error": (ctypes.c_char_p, []),
    "hb_version": (_c_int, []),
    "hb_stream_capture_id": (_c_int, [_p, _p]),
    "hb_attention_workspace_bytes": (_c_i64, [_c_int] * 9),
    "hb_paired_fwd": (
        _c_int,
        [_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _c_int, _c_int,
         _c_int, _c_int, _c_f32, _p, _c_i64, _c_int, _p],
    ),
    "hb_paired_fwd_noalloc": (
        _c_int,
        [_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _c_int, _c_int,
         _c_int, _c_int, _c_f32, _c_int, _p],
    ),
    "hb_quad_fwd": (
        _c_int,
        [_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _c_int, _c_int,
         _c_int, _c_f32, _p, _c_i64, _c_int, _p],
    ),
    "hb_block_sparse_fwd": (
        _c_int,
        [_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _c_int, _c_int,
         _c_int, _c_int, _c_f32, _p, _c_i64, _c_int, _p],
    ),
    "hb_gather_rows": (
        _c_int, [_p, _p, _p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _p, _p],
    ),
    "hb_qk_prep": (
        _c_int,
        [_p, _p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _p, _c_f32, _p, _p, _p, _c_i64, _c_i64, _c_i64, _p],
    ),
    "hb_adaln_modulate": (
        _c_int,
        [_c_int, _c_int, _c_int, _c_int, _c_f32, _p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _c_i64,
         _p, _c_i64, _c_i64, _p, _p, _c_i64, _p, _c_i64, _c_i64, _p],
    ),
    "hb_hilbert_order": (_c_int, [_c_int, _p, _p]),
    "hb_plan_layout": (_c_int, [_c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _p, _p, _p, _p]),
    "hb_plan_scratch_bytes": (_c_i64, [_c_int, _c_int]),
    "hb_plan_phase_bits": (
        _c_int,
        [_p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p],
    ),
    "hb_table_bits": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _p, _p]),
    "hb_bits_counts": (_c_int, [_p, _c_int, _c_int, _c_int, _p, _p, _p, _p]),
    "hb_bits_emit": (_c_int, [_p, _c_int, _c_int, _c_int, _p, _c_int, _p, _p, _c_int, _p]),
    "hb_pair_rows": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _c_int, _p, _p]),
    "hb_quad_rows": (_c_int, [_p, _p, _p, _c_int, _c_int, _c_int, _p, _p, _p, _c_int, _p, _p]),
    "hb_mfma_peak_probe": (_c_int, [_c_int, _c_int, _p, _p, _p]),
    "hb_paired_plan_scratch_bytes": (_c_i64, [_c_int, _c_int]),
    "hb_paired_plan_tables": (
        _c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    ),
    "hb_paired_plan_emit": (_c_int, [_c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _p, _p]),
    "hb_hilbert_order_host": (_c_int, [_c_int, _p]),
    "hb_plan_layout_host": (_c_int, [_c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _p, _p, _p]),
    "hb_plan_phase_bits_host": (
        _c_int,
        [_p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p],
    ),
    "hb_table_bits_host": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _p]),
    "hb_bits_counts_host": (_c_int, [_p, _c_int, _c_int, _c_int, _p, _p, _p]),
    "hb_bits_emit_host": (_c_int, [_p, _c_int, _c_int, _c_int, _p, _c_int, _p, _p, _c_int]),
    "hb_pair_rows_host": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _c_int, _p]),
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/hilberta_hip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(hb_\w+)\s*\(", text, re.M)))


def header_abi_version() -> int:
    """HB_ABI_VERSION as include/hilberta_hip.h defines it."""
    m = re.search(r"^#define\s+HB_ABI_VERSION\s+(\d+)", HEADER.read_text(), re.M)
    if not m:
        raise RuntimeError(f"{HEADER} defines no HB_ABI_VERSION")
    return int(m.group(1))


def load():
    """Load the library (once) and declare its signatures; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first (python -m hilberta_amd.build); "
                "there is no CPU fallback"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.hb_version.restype = ctypes.c_int32
        built, declared = lib.hb_version(), header_abi_version()
        if built != declared:
            raise RuntimeError(
                f"{LIB_PATH} was built for ABI {built} but include/hilberta_hip.h declares ABI "
                f"{declared}: rebuild the HIP library (python -m hilberta_amd.build)"
            )
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def last_error() -> str:
    return (load().hb_last_error() or b"").decode(errors="replace")


def check(rc: int, name: str) -> None:
    if rc == 0:
        return
    msg = f"{name}: {last_error()}"
    if rc == HB_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def stream_ptr(device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors) -> None:
    for t in tensors:
        if not (isinstance(t, torch.Tensor) and t.is_cuda):
            raise ValueError("HIP entry points take device tensors on one CUDA (HIP) device")
