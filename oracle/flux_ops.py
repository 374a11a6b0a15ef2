"""FLUX attention-input formulas (QK RMSNorm, rotary embedding, position tables) -- TEST ORACLE ONLY.

The reference calls these from diffusers, a dependency that is absent here: diffusers==0.36.0
(pinned at reference requirements-cu126.txt:6 and pyproject.toml:9).  The call sites are
hilberta/flux_adapter.py:283-295 (attn.norm_q / norm_k / norm_added_q / norm_added_k, the
torch.cat of text and image tokens, apply_rotary_emb) and :17 (the apply_rotary_emb import).
Their published algorithms, restated:

  * RMSNorm (diffusers.models.normalization.RMSNorm, elementwise_affine, eps 1e-6 in FLUX):
      var = mean(float32(x)^2 over head_dim);  y = float32(x) * rsqrt(var + eps)
      y = y.to(weight dtype) * weight   (bf16 multiply)   -- or y.to(x dtype) without weight
  * apply_rotary_emb(x, (cos, sin), use_real=True, use_real_unbind_dim=-1, sequence_dim=1):
      pairs (x[2i], x[2i+1]);  rot = (-x[2i+1], x[2i]) interleaved
      out = (float32(x) * cos + float32(rot) * sin).to(x dtype)
  * FluxPosEmbed(theta=10000, axes_dim=(16, 56, 56)) over ids [N, 3]:
      per axis a of width d: freq_j = 1 / theta^(2j/d) (float64), angle = pos_a * freq_j,
      cos/sin repeated twice (interleaved) -> d columns; axes concatenated -> 128; float32.

Pinned by (tests/test_oracle_flux_ops.py): the rotation equals complex multiplication by
exp(i * angle) on (x[2i] + i x[2i+1]) (torch.polar / view_as_complex, a different formulation);
position 0 is the identity; rotating by a then b equals rotating by a + b; RMSNorm of a constant
row is sign(x) * w / sqrt(1 + eps) and of a one-hot row sqrt(128 / (1 + 128 eps)) at the hot
index; the frequency table equals a float64 loop over its definition; pair norms are preserved.
"""

from __future__ import annotations

import math

import torch

THETA = 10000
AXES_DIM = (16, 56, 56)


def rms_norm(x, weight=None, eps=1e-6):
    """diffusers 0.36.0 RMSNorm.forward over the last dimension (x bf16/fp16, weight same dtype)."""
    var = x.float().pow(2).mean(-1, keepdim=True)
    y = x.float() * torch.rsqrt(var + eps)
    if weight is None:
        return y.to(x.dtype)
    return y.to(weight.dtype) * weight


def rotate_pairs(x):
    """(x0, x1, x2, x3, ...) -> (-x1, x0, -x3, x2, ...) over the last dimension."""
    re, im = x.unflatten(-1, (-1, 2)).unbind(-1)
    return torch.stack([-im, re], dim=-1).flatten(-2)


def apply_rotary(x, cos, sin):
    """apply_rotary_emb(use_real=True, use_real_unbind_dim=-1) for x [B, N, H, D], cos/sin [N, D]."""
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return (x.float() * c + rotate_pairs(x).float() * s).to(x.dtype)


def rotary_tables(ids, theta=THETA, axes_dim=AXES_DIM):
    """FluxPosEmbed.forward: ids [N, 3] -> (cos, sin) float32 [N, sum(axes_dim)]."""
    pos = ids.float()
    cos_parts, sin_parts = [], []
    for axis, dim in enumerate(axes_dim):
        freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64, device=ids.device) / dim))
        angles = torch.outer(pos[:, axis].double(), freqs)
        cos_parts.append(angles.cos().repeat_interleave(2, dim=1).float())
        sin_parts.append(angles.sin().repeat_interleave(2, dim=1).float())
    return torch.cat(cos_parts, dim=-1), torch.cat(sin_parts, dim=-1)


def rotary_tables_loop(ids, theta=THETA, axes_dim=AXES_DIM):
    """The same tables from a float64 per-entry loop over the definition (tiny inputs only)."""
    n = ids.shape[0]
    width = sum(axes_dim)
    cos = torch.zeros(n, width, dtype=torch.float64)
    sin = torch.zeros(n, width, dtype=torch.float64)
    for t in range(n):
        col = 0
        for axis, dim in enumerate(axes_dim):
            p = float(torch.tensor(float(ids[t, axis]), dtype=torch.float32))
            for j in range(dim // 2):
                angle = p * (1.0 / theta ** (2 * j / dim))
                cos[t, col + 2 * j] = cos[t, col + 2 * j + 1] = math.cos(angle)
                sin[t, col + 2 * j] = sin[t, col + 2 * j + 1] = math.sin(angle)
            col += dim
    return cos.float(), sin.float()


def flux_ids(text_tokens, grid):
    """FLUX position ids: text rows all zero; image row (r, c) of a grid x grid latent -> (0, r, c)
    (diffusers FluxPipeline._prepare_latent_image_ids), in raster order."""
    txt = torch.zeros(text_tokens, 3)
    r, c = torch.meshgrid(torch.arange(grid), torch.arange(grid), indexing="ij")
    img = torch.stack([torch.zeros(grid * grid), r.reshape(-1).float(), c.reshape(-1).float()], -1)
    return txt, img


def qk_prep(text, image, *, heads, weight_text=None, weight_image=None, eps=1e-6, cos=None,
            sin=None, normalize=True):
    """The processor's sequence for one of Q/K (flux_adapter.py:283-295): per-head RMSNorm of the
    image and text projections with their own weights, [text; image] concatenation, rotation.
    text [B, T, H*D], image [B, n, H*D] -> [B, T+n, H, D]."""
    t = text.unflatten(-1, (heads, -1))
    i = image.unflatten(-1, (heads, -1))
    if normalize:
        t = rms_norm(t, weight_text, eps)
        i = rms_norm(i, weight_image, eps)
    x = torch.cat([t, i], dim=1)
    if cos is not None:
        x = apply_rotary(x, cos, sin)
    return x
