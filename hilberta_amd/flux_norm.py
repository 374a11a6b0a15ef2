"""Gated residual + AdaLN modulation of the FLUX blocks in one HIP pass (csrc/adaln.hip).

``adaln_modulate(x, shift, scale, y=y, gate=gate, x_out=x)`` computes, per token row,

    r = x + gate * y;  x_out = r;  out = shift + LayerNorm(r) * (1 + scale)

which the FLUX blocks (diffusers 0.36.0 FluxTransformerBlock / FluxSingleTransformerBlock with
AdaLayerNormZero / AdaLayerNormZeroSingle / AdaLayerNormContinuous) run as separate torch passes:
``torch.addcmul`` for the gated residual, ``layer_norm``, ``1 + scale`` and another ``addcmul``.
"""

from __future__ import annotations

import torch

from . import _lib

_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def _rows(t, name, B, R, C):
    if t.ndim != 3 or t.shape != (B, R, C) or t.stride(-1) != 1:
        raise ValueError(f"{name} must be [B, rows, hidden] with a contiguous last dimension")
    return t.stride(0), t.stride(1)


def adaln_modulate(x, shift, scale, *, y=None, gate=None, x_out=None, out=None, eps=1e-6):
    """x [B, rows, hidden]; shift / scale / gate [B, hidden] (views with a contiguous last dim,
    e.g. chunks of one modulation projection); y like x.  Returns out [B, rows, hidden]."""
    _lib.require_gpu(x)
    if x.dtype not in _DTYPES:
        raise ValueError("adaln_modulate takes bf16 or fp16 rows")
    B, R, C = x.shape if x.ndim == 3 else (0, 0, 0)
    xb, xn = _rows(x, "x", B, R, C)
    yb = yn = ob = on = 0
    if (y is None) != (gate is None):
        raise ValueError("y and gate are given together")
    if x_out is not None and y is None:
        raise ValueError("x_out is written only with a residual update")
    mods = [shift, scale] + ([gate] if gate is not None else [])
    for m in mods:
        if m.ndim != 2 or m.shape != (B, C) or m.stride(-1) != 1 or m.dtype != x.dtype:
            raise ValueError("shift/scale/gate must be [B, hidden] views with a contiguous last dim")
    mod_b = shift.stride(0)
    if scale.stride(0) != mod_b:
        raise ValueError("shift and scale must share one batch stride")
    tensors = [x] + mods
    if y is not None:
        yb, yn = _rows(y, "y", B, R, C)
        tensors.append(y)
    if x_out is not None:
        ob, on = _rows(x_out, "x_out", B, R, C)
        tensors.append(x_out)
    if out is None:
        out = torch.empty(B, R, C, dtype=x.dtype, device=x.device)
    pb, pn = _rows(out, "out", B, R, C)
    tensors.append(out)
    if any(t.device != x.device or t.dtype != x.dtype for t in tensors):
        raise ValueError("all tensors must share x's device and dtype")
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = _lib.load().hb_adaln_modulate(
        B, R, C, _DTYPES[x.dtype], float(eps), x.data_ptr(), xb, xn, ptr(y), yb, yn, ptr(gate),
        gate.stride(0) if gate is not None else 0, ptr(x_out), ob, on, shift.data_ptr(), scale.data_ptr(), mod_b, out.data_ptr(), pb, pn,
        _lib.stream_ptr(x.device),
    )
    _lib.check(rc, "hb_adaln_modulate")
    return out
