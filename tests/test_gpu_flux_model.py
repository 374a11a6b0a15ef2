"""GPU checks of the FLUX-shaped transformer with the persistent layout and the HIP attention.

Mirrors the reference's whole-transformer gates (tests/test_adapter.py:314-355) on a shallow model
of the real head size (2 double + 3 single blocks, 4 heads x 128, so layer phases 0,1,2,3,0):

  * persistent layout + paired kernel on the plan's tables equals the raster-order model whose
    attention applies each phase's mask scattered to raster token identities (an independent
    formulation: torch SDPA with an explicit boolean mask, no permutation anywhere);
  * persistent layout on all-connection tables equals the raster model with dense attention
    (permutation equivalence);
  * the unpaired kernel and the dense-mask backend agree with the paired kernel in the layout.

Tolerance: relative L2 error of the bf16 prediction <= 2e-2 (the reference's correctness gate for
attention outputs, hilberta/benchmark.py:73-75), here after five blocks of bf16 arithmetic.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import say

pytestmark = pytest.mark.gpu

REL_L2 = 2e-2


def _rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm())


class RasterMaskAttention:
    """Raster token order; layer i attends with phase i % 4 of the plan scattered to raster
    identities (test_adapter.py:63-73)."""

    layout = None

    def __init__(self, plan, device):
        T = plan.text_tokens
        identity = torch.cat([torch.arange(T), T + plan.image_order.cpu().long()])
        self.masks = []
        for phase in range(4):
            dense = torch.zeros(plan.total_tokens, plan.total_tokens, dtype=torch.bool)
            dense[identity[:, None], identity[None, :]] = plan.dense_mask(phase, "cpu")
            assert dense[:T].all() and dense[:, :T].all()
            self.masks.append(dense.to(device))
        self.phases = []

    def __call__(self, layer, q, k, v, out):
        self.phases.append(layer % 4)
        out.copy_(F.scaled_dot_product_attention(q, k, v, attn_mask=self.masks[layer % 4]))


@pytest.fixture(scope="module")
def small(hip_device):
    from hilberta_amd.flux_model import FluxShape, FluxTransformer, synthetic_inputs

    shape = FluxShape(num_layers=2, num_single_layers=3, heads=4)
    model = FluxTransformer(hip_device, shape, seed=1)
    args = synthetic_inputs(hip_device, grid=64, shape=shape, seed=2)
    return model, args


@pytest.mark.parametrize("tiles,k", [(4, 1), (16, 3)])
def test_persistent_paired_equals_raster_masked_reference(hip_device, small, tiles, k):
    from hilberta_amd.bridge_k import bridge_k_plan
    from hilberta_amd.flux_model import PersistentAttention

    model, args = small
    plan = bridge_k_plan(tiles, k, False, grid_size=64)
    say(f"case flux model paired t{tiles}k{k} vs raster masks")
    reference_attn = RasterMaskAttention(plan, hip_device)
    reference = model(**args, attention=reference_attn)
    paired = PersistentAttention(plan, hip_device, "paired")
    actual = model(**args, attention=paired)
    torch.cuda.synchronize()
    assert reference_attn.phases == [0, 1, 2, 3, 0] and paired.calls == 5
    assert actual.shape == args["hidden_states"].shape and bool(torch.isfinite(actual).all())
    err = _rel(actual, reference)
    say(f"  relative L2 {err:.3e}")
    assert err <= REL_L2


def test_full_tables_layout_equals_native_dense(hip_device, small):
    from hilberta_amd.bridge_k import bridge_k_plan
    from hilberta_amd.flux_model import NativeAttention, PersistentAttention
    from hilberta_amd.plan import full_attention_plan

    model, args = small
    plan = full_attention_plan(bridge_k_plan(16, 3, False, grid_size=64))
    say("case flux model full tables in layout vs native dense")
    native = model(**args, attention=NativeAttention())
    reordered = model(**args, attention=PersistentAttention(plan, hip_device, "paired"))
    torch.cuda.synchronize()
    err = _rel(reordered, native)
    say(f"  relative L2 {err:.3e}")
    assert err <= REL_L2


def test_backends_agree_in_layout(hip_device, small):
    from hilberta_amd.bridge_k import bridge_k_plan
    from hilberta_amd.flux_model import PersistentAttention

    model, args = small
    plan = bridge_k_plan(16, 3, False, grid_size=64)
    say("case flux model paired / sparse / sdpa_reference backends")
    out = {b: model(**args, attention=PersistentAttention(plan, hip_device, b))
           for b in ("paired", "sparse", "sdpa_reference")}
    torch.cuda.synchronize()
    assert _rel(out["sparse"], out["paired"]) <= REL_L2
    assert _rel(out["paired"], out["sdpa_reference"]) <= REL_L2


def test_device_plan_equals_host_plan(hip_device, small):
    """The all-device plan (paired_plan_device) drives the same computation bit for bit."""
    from hilberta_amd.bridge_k import bridge_k_plan, paired_plan_device
    from hilberta_amd.flux_model import PersistentAttention

    model, args = small
    say("case flux model device plan vs host plan")
    a = model(**args, attention=PersistentAttention(bridge_k_plan(4, 1, False, grid_size=64), hip_device))
    b = model(**args, attention=PersistentAttention(paired_plan_device(4, 1, grid_size=64, device=hip_device),
                                                    hip_device))
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_full_size_model_parameter_count_and_step(hip_device):
    """The FLUX.1-dev-shaped model holds exactly the analytic parameter count and one 1024 px
    denoiser step through the paired kernel gives a finite prediction."""
    from hilberta_amd.bridge_k import paired_plan_device
    from hilberta_amd.flux_model import FluxTransformer, PersistentAttention, synthetic_inputs
    from tests.test_flux_shape import flux_dev_parameter_count

    say("case full-size FLUX-shaped model 1024 px")
    model = FluxTransformer(hip_device, seed=3)
    assert model.parameter_count() == flux_dev_parameter_count()
    args = synthetic_inputs(hip_device, grid=64, seed=4)
    attn = PersistentAttention(paired_plan_device(16, 3, grid_size=64, device=hip_device), hip_device)
    out = model(**args, attention=attn)
    torch.cuda.synchronize()
    assert attn.calls == 57 and bool(torch.isfinite(out).all())
    say(f"  prediction std {float(out.float().std()):.3f}")
    del model
    torch.cuda.empty_cache()
