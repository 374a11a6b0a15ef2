"""GPU checks of the sampling-scope layout (reference tests/test_sampling_layout.py:54-123): one
entry and one exit permutation for a whole trajectory gives the same bits as permuting at every
transformer call, and with all-connection tables the persistent layout matches the raster model."""

import pytest
import torch

from tests.helpers import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(hip_device):
    from hilberta_amd.flux_model import FluxShape, FluxTransformer, synthetic_inputs

    shape = FluxShape(num_layers=1, num_single_layers=2, heads=4)
    model = FluxTransformer(hip_device, shape, seed=5)
    args = synthetic_inputs(hip_device, grid=64, shape=shape, seed=6)
    return model, args


def _run(model, args, attention, scope, steps=3):
    from hilberta_amd.sampling_layout import sample_flux

    return sample_flux(model, args["hidden_states"], args["encoder_hidden_states"],
                       args["pooled_projections"], args["img_ids"], args["txt_ids"], steps=steps,
                       attention=attention, layout_scope=scope)


def test_sampling_scope_matches_per_forward_bitwise(hip_device, small):
    from hilberta_amd.bridge_k import paired_plan_device
    from hilberta_amd.flux_model import PersistentAttention

    model, args = small
    attention = PersistentAttention(paired_plan_device(16, 3, grid_size=64, device=hip_device), hip_device)
    say("case sampling scope vs transformer scope, 3 steps")
    per_forward, info_t = _run(model, args, attention, "transformer")
    once, info_s = _run(model, args, attention, "sampling")
    torch.cuda.synchronize()
    assert torch.equal(once, per_forward)
    assert info_s["sampling_image_reorder_calls"] == info_s["sampling_inverse_calls"] == 1
    assert info_s["sampling_id_reorder_calls"] == 1 and info_s["transformer_calls"] == 3
    assert info_t["sampling_image_reorder_calls"] == info_t["sampling_inverse_calls"] == 0
    n = args["hidden_states"].shape[1]
    assert info_s["sampling_layout_read_write_bytes"] == 2 * (n * 64 * 2 + n * 3 * 4) + 2 * n * 64 * 2


def test_full_tables_sampling_matches_raster(hip_device, small):
    from hilberta_amd.bridge_k import bridge_k_plan
    from hilberta_amd.flux_model import NativeAttention, PersistentAttention
    from hilberta_amd.plan import full_attention_plan

    model, args = small
    say("case full tables, sampling scope vs raster dense attention")
    raster, _ = _run(model, args, NativeAttention(), "sampling")
    plan = full_attention_plan(bridge_k_plan(16, 3, False, grid_size=64))
    packed, _ = _run(model, args, PersistentAttention(plan, hip_device, "paired"), "sampling")
    torch.cuda.synchronize()
    err = float((packed.float() - raster.float()).norm() / raster.float().norm())
    say(f"  relative L2 {err:.3e}")
    assert err <= 2e-2


def test_rejects_unknown_scope(hip_device, small):
    model, args = small
    with pytest.raises(ValueError):
        _run(model, args, None, "image")
