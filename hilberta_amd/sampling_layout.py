"""One entry / exit permutation for a whole FLUX sampling trajectory (reference
hilberta/sampling_layout.py:20-148), on the FLUX-shaped transformer of flux_model.py.

The reference wraps diffusers' FluxPipeline: it gathers the prepared latents and image ids into
the plan's order once after ``prepare_latents`` (sampling_layout.py:88-103), runs every
transformer call with ``layout_scope="sampling"`` (no per-call permutation, flux_adapter.py:
205-220), and gathers the final latents back to raster order once before ``_unpack_latents``
(:105-116).  The scheduler's Euler update is elementwise per token, so it runs unchanged on the
packed latents.  diffusers is absent here, so the loop is restated from FluxPipeline.__call__ with
FLUX.1-dev's FlowMatchEulerDiscreteScheduler configuration (diffusers 0.36.0):

  sigmas_i = linspace(1, 1/steps, steps);  mu = calculate_shift(image tokens)
  sigma_i  = exp(mu) / (exp(mu) + (1/sigma_i - 1))          (exponential time shift)
  timestep = bf16(1000 sigma_i) / 1000 passed to the transformer
  latents  = bf16(f32(latents) + (sigma_{i+1} - sigma_i) f32(prediction)),  sigma_steps = 0

The permutations run on the HIP gather (layout.index_select_rows); counters mirror the
reference's boundary dictionary.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .layout import index_select_rows

# FLUX.1-dev scheduler configuration (scheduler_config.json of the model repository)
BASE_IMAGE_SEQ_LEN = 256
MAX_IMAGE_SEQ_LEN = 4096
BASE_SHIFT = 0.5
MAX_SHIFT = 1.15
NUM_TRAIN_TIMESTEPS = 1000


def calculate_shift(image_seq_len, base_seq_len=BASE_IMAGE_SEQ_LEN, max_seq_len=MAX_IMAGE_SEQ_LEN,
                    base_shift=BASE_SHIFT, max_shift=MAX_SHIFT):
    """FluxPipeline's calculate_shift: mu linear in the image token count."""
    m = (max_shift - base_shift) / (max_seq_len - base_seq_len)
    b = base_shift - m * base_seq_len
    return image_seq_len * m + b


def flux_sigmas(steps, image_seq_len):
    """float32 sigmas [steps + 1] (terminal 0) of FlowMatchEulerDiscreteScheduler.set_timesteps
    with dynamic exponential shifting, and the float32 timesteps (1000 sigma) [steps]."""
    if steps < 1:
        raise ValueError("steps must be positive")
    base = np.linspace(1.0, 1 / steps, steps)
    mu = calculate_shift(image_seq_len)
    shifted = math.exp(mu) / (math.exp(mu) + (1 / base - 1) ** 1.0)
    sigmas = torch.from_numpy(shifted).to(torch.float32)
    timesteps = sigmas * NUM_TRAIN_TIMESTEPS
    return torch.cat([sigmas, torch.zeros(1)]), timesteps


@torch.inference_mode()
def sample_flux(model, latents, encoder_hidden_states, pooled_projections, img_ids, txt_ids, *,
                steps, guidance=3.5, attention=None, layout_scope="sampling"):
    """Run ``steps`` denoising steps of ``model`` from raster-order packed ``latents`` [B, n, 64];
    returns (final raster-order latents, info).

    With a persistent-layout ``attention`` and ``layout_scope="sampling"`` the image tokens and
    ids are permuted once here; with ``"transformer"`` every transformer call permutes at its own
    entry and exit (flux_adapter.py:209-212, :243).  Without a layout both run in raster order.
    """
    if layout_scope not in ("transformer", "sampling"):
        raise ValueError("layout_scope must be transformer or sampling")
    layout = getattr(attention, "layout", None)
    B, n, _ = latents.shape
    sigmas, timesteps = flux_sigmas(steps, n)
    info = dict(sampling_image_reorder_calls=0, sampling_id_reorder_calls=0,
                sampling_inverse_calls=0, sampling_layout_read_write_bytes=0, transformer_calls=0,
                layout_scope=layout_scope)
    packed = layout is not None and layout_scope == "sampling"
    if packed:
        latents = index_select_rows(latents, 1, layout.order)
        img_ids = index_select_rows(img_ids.contiguous(), 0, layout.order)
        info["sampling_image_reorder_calls"] += 1
        info["sampling_id_reorder_calls"] += 1
        info["sampling_layout_read_write_bytes"] += 2 * (latents.numel() * latents.element_size()
                                                         + img_ids.numel() * img_ids.element_size())
    guidance_t = torch.full((B,), guidance, device=latents.device, dtype=torch.float32)
    for i in range(steps):
        t = timesteps[i].expand(B).to(latents.device)
        pred = model(latents, encoder_hidden_states, pooled_projections,
                     t.to(latents.dtype) / NUM_TRAIN_TIMESTEPS, img_ids, txt_ids, guidance_t,
                     attention=attention, layout_scope=layout_scope)
        info["transformer_calls"] += 1
        step = float(sigmas[i + 1] - sigmas[i])
        latents = (latents.float() + step * pred.float()).to(pred.dtype)
    if packed:
        latents = index_select_rows(latents, 1, layout.inverse)
        info["sampling_inverse_calls"] += 1
        info["sampling_layout_read_write_bytes"] += 2 * latents.numel() * latents.element_size()
    return latents, info
