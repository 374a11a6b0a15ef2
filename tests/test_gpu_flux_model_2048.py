"""FLUX-shaped denoiser step at 2048 px (128 x 128 latent grid, 16384 image + 512 text tokens).

  * The shallow model's gates of test_gpu_flux_model.py at grid 128: persistent layout + paired
    kernel against the raster-order model whose attention applies each phase's mask scattered to
    raster token identities, for 16-tile K3 and 4-tile K1 plans.
  * The full-size FLUX.1-dev-shaped model (19 double + 38 single blocks, 24 heads x 128), one
    denoiser step at 2048 px through the paired kernel against the same model with the
    dense-mask SDPA backend (the adapter's sdpa_reference backend, flux_adapter.py:300-306):
    finite, 57 attention calls, relative L2 <= 2e-2.

Reference rows of this step: results/efficiency_all_rows.csv:162 (full), :192 (16-tile K3),
:204 (4-tile K1).
"""

import pytest
import torch

from tests.helpers import say
from tests.test_gpu_flux_model import REL_L2, RasterMaskAttention, _rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small_2048(hip_device):
    from hilberta_amd.flux_model import FluxShape, FluxTransformer, synthetic_inputs

    shape = FluxShape(num_layers=2, num_single_layers=3, heads=4)
    model = FluxTransformer(hip_device, shape, seed=11)
    args = synthetic_inputs(hip_device, grid=128, shape=shape, seed=12)
    return model, args


@pytest.mark.parametrize("tiles,k", [(16, 3), (4, 1)])
def test_small_model_2048_paired_equals_raster_masked(hip_device, small_2048, tiles, k):
    from hilberta_amd.bridge_k import bridge_k_plan
    from hilberta_amd.flux_model import PersistentAttention

    model, args = small_2048
    plan = bridge_k_plan(tiles, k, False, grid_size=128)
    say(f"case flux model 2048 px paired t{tiles}k{k} vs raster masks")
    reference_attn = RasterMaskAttention(plan, hip_device)
    reference = model(**args, attention=reference_attn)
    paired = PersistentAttention(plan, hip_device, "paired")
    actual = model(**args, attention=paired)
    torch.cuda.synchronize()
    assert reference_attn.phases == [0, 1, 2, 3, 0] and paired.calls == 5
    assert bool(torch.isfinite(actual).all())
    err = _rel(actual, reference)
    say(f"  relative L2 {err:.3e}")
    assert err <= REL_L2
    del reference_attn
    torch.cuda.empty_cache()


def test_full_size_model_2048_step(hip_device):
    from hilberta_amd.bridge_k import bridge_k_plan, paired_plan_device
    from hilberta_amd.flux_model import FluxTransformer, PersistentAttention, synthetic_inputs

    say("case full-size FLUX-shaped model 2048 px: paired vs dense-mask SDPA backend")
    model = FluxTransformer(hip_device, seed=13)
    args = synthetic_inputs(hip_device, grid=128, seed=14)
    paired = PersistentAttention(paired_plan_device(16, 3, grid_size=128, device=hip_device), hip_device)
    actual = model(**args, attention=paired)
    reference_attn = PersistentAttention(bridge_k_plan(16, 3, False, grid_size=128), hip_device,
                                         "sdpa_reference")
    reference = model(**args, attention=reference_attn)
    torch.cuda.synchronize()
    assert paired.calls == 57 and reference_attn.calls == 57
    assert actual.shape == args["hidden_states"].shape
    assert bool(torch.isfinite(actual).all()) and bool(torch.isfinite(reference).all())
    err = _rel(actual, reference)
    say(f"  relative L2 {err:.3e}, prediction std {float(actual.float().std()):.3f}")
    assert err <= REL_L2
    del model, reference_attn
    torch.cuda.empty_cache()
