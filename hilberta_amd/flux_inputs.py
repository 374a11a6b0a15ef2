"""FLUX attention inputs on the GPU: QK RMSNorm + rotary embedding + [text; image] BNHD write.

Replaces the sequence the reference's attention processor runs between the Q/K/V projections and
the attention call (hilberta/flux_adapter.py:283-295): diffusers' ``attn.norm_q`` / ``norm_k`` /
``norm_added_q`` / ``norm_added_k`` (RMSNorm over each 128-wide head), ``torch.cat`` of the text
and image tokens and ``apply_rotary_emb`` -- one HIP pass (csrc/qk_prep.hip) per tensor instead
of five to eight torch kernels.  The output is the [B, N, H, D] storage that the attention kernels
read as a [B, H, N, D] view (``.transpose(1, 2)``), so no further copy is made.

``rotary_tables`` builds FluxPosEmbed's (cos, sin) rows (theta 10000, axes 16/56/56) for the ids
in the order the tokens are stored, e.g. after the persistent Hilbert permutation of the image ids
(flux_adapter.py:210-212).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

HEAD_DIM = 128
THETA = 10000
AXES_DIM = (16, 56, 56)
_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def rotary_tables(ids, theta=THETA, axes_dim=AXES_DIM):
    """(cos, sin) float32 [N, 128] for position ids [N, 3] (diffusers 0.36.0 FluxPosEmbed: float64
    angles pos * theta^(-2j/d) per axis, each value repeated for the pair, axes concatenated)."""
    if ids.ndim != 2 or ids.shape[1] != len(axes_dim) or sum(axes_dim) != HEAD_DIM:
        raise ValueError("ids must be [N, 3] and the axes must add up to 128")
    pos = ids.to(torch.float32).to(torch.float64)
    cos, sin = [], []
    for axis, dim in enumerate(axes_dim):
        exponent = torch.arange(0, dim, 2, dtype=torch.float64, device=ids.device) / dim
        angles = pos[:, axis, None] * (1.0 / theta**exponent)[None, :]
        cos.append(angles.cos().repeat_interleave(2, dim=1))
        sin.append(angles.sin().repeat_interleave(2, dim=1))
    return (torch.cat(cos, 1).to(torch.float32).contiguous(),
            torch.cat(sin, 1).to(torch.float32).contiguous())


def _rows(x, name):
    if x.ndim != 3 or x.stride(-1) != 1:
        raise ValueError(f"{name} must be [B, tokens, columns] with a contiguous last dimension")
    return x.stride(0), x.stride(1)


def _launch(text, image, *, heads, planes, out, out_plane_stride, normalize, weights, eps, cos, sin):
    _lib.require_gpu(image)
    width = planes * heads * HEAD_DIM
    if image.ndim != 3 or image.shape[2] != width:
        raise ValueError(f"image must be [B, n, {planes}*heads*128]")
    B, n = image.shape[:2]
    T = 0 if text is None else text.shape[1]
    if text is not None:
        _lib.require_gpu(text)
        if text.ndim != 3 or text.shape[0] != B or text.shape[2] != width or text.dtype != image.dtype:
            raise ValueError("text must be [B, T, columns] with image's batch, columns and dtype")
    if image.dtype not in _DTYPES:
        raise ValueError("Q/K/V projections must be bf16 or fp16")
    N = T + n
    plane_shape = (B, N, heads, HEAD_DIM)
    views = [out] if planes == 1 else [out[0], out[1]]
    for o in views:
        if o.shape != plane_shape or o.dtype != image.dtype or o.stride(3) != 1 or o.stride(2) != HEAD_DIM:
            raise ValueError("out must be [B, N, heads, 128] per plane with contiguous heads")
    tensors = [image, out] + ([text] if text is not None else [])
    flat = [w for pair in weights for w in pair]
    for w in flat:
        if w is not None:
            if not normalize or w.shape != (HEAD_DIM,) or w.dtype != image.dtype or not w.is_contiguous():
                raise ValueError("norm weights are contiguous [128] tensors in the input dtype")
            tensors.append(w)
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must be given together")
    if cos is not None:
        for c in (cos, sin):
            if c.shape != (N, HEAD_DIM) or c.dtype != torch.float32 or not c.is_contiguous():
                raise ValueError("cos/sin must be contiguous float32 [N, 128]")
            tensors.append(c)
    if any(t.device != image.device for t in tensors):
        raise ValueError("all tensors must be on one device")
    tb, tr = _rows(text, "text") if text is not None else (0, 0)
    ib, ir = _rows(image, "image")
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    warr = (ctypes.c_void_p * 4)(*[ptr(w) for w in flat], *([None] * (4 - len(flat))))
    o0 = views[0]
    rc = _lib.load().hb_qk_prep(
        ptr(text), image.data_ptr(), tb, tr, ib, ir, planes, heads * HEAD_DIM, B, T, N, heads,
        HEAD_DIM, _DTYPES[image.dtype], int(bool(normalize)), warr, float(eps), ptr(cos), ptr(sin),
        o0.data_ptr(), out_plane_stride, o0.stride(0), o0.stride(1), _lib.stream_ptr(image.device),
    )
    _lib.check(rc, "hb_qk_prep")
    return out


def _new_out(planes, text, image, heads):
    B, n = image.shape[:2]
    N = n + (0 if text is None else text.shape[1])
    shape = (B, N, heads, HEAD_DIM) if planes == 1 else (2, B, N, heads, HEAD_DIM)
    return torch.empty(shape, dtype=image.dtype, device=image.device)


def qk_prep(text, image, *, heads, out=None, normalize=True, weight_text=None, weight_image=None,
            eps=1e-6, cos=None, sin=None):
    """[text; image] tokens -> out [B, T+n, heads, 128], with per-head RMSNorm (weights optional)
    when ``normalize`` and the rotation when ``cos``/``sin`` are given.

    ``text`` [B, T, heads*128] and ``image`` [B, n, heads*128] may be column slices of a fused
    projection (row stride > heads*128) or row ranges of one tensor.  ``text`` may be None (T = 0).
    """
    if out is None:
        out = _new_out(1, text, image, heads)
    return _launch(text, image, heads=heads, planes=1, out=out, out_plane_stride=0,
                   normalize=normalize, weights=((weight_text, weight_image),), eps=eps, cos=cos,
                   sin=sin)


def qk_prep_pair(text, image, *, heads, out=None, weights=((None, None), (None, None)), eps=1e-6,
                 cos=None, sin=None):
    """Q and K in one launch: ``text`` / ``image`` hold the Q columns then the K columns
    ([B, T or n, 2*heads*128], e.g. a slice of a fused QKV projection); both are RMS-normalised
    with ``weights`` = ((q_text, q_image), (k_text, k_image)) and rotated.  Returns out
    [2, B, N, heads, 128] (out[0] = Q, out[1] = K)."""
    if out is None:
        out = _new_out(2, text, image, heads)
    if out.ndim != 5 or out.shape[0] != 2:
        raise ValueError("out must be [2, B, N, heads, 128]")
    return _launch(text, image, heads=heads, planes=2, out=out, out_plane_stride=out.stride(0),
                   normalize=True, weights=weights, eps=eps, cos=cos, sin=sin)
