"""CPU checks of the FLUX flow-matching schedule restated in hilberta_amd/sampling_layout.py
(diffusers 0.36.0 FluxPipeline.calculate_shift and FlowMatchEulerDiscreteScheduler with dynamic
exponential shifting): closed forms at the configuration's end points and invariants."""

import math

import pytest
import torch

from hilberta_amd.sampling_layout import calculate_shift, flux_sigmas


def test_shift_end_points_and_linearity():
    assert calculate_shift(256) == pytest.approx(0.5)
    assert calculate_shift(4096) == pytest.approx(1.15)
    assert calculate_shift(2176) == pytest.approx((0.5 + 1.15) / 2)


@pytest.mark.parametrize("steps,n", [(1, 4096), (4, 4096), (28, 16384), (50, 1024)])
def test_sigmas_shape_and_invariants(steps, n):
    sigmas, timesteps = flux_sigmas(steps, n)
    assert sigmas.shape == (steps + 1,) and timesteps.shape == (steps,)
    assert sigmas.dtype == torch.float32 and float(sigmas[0]) == 1.0 and float(sigmas[-1]) == 0.0
    assert bool((sigmas[1:] < sigmas[:-1]).all())
    assert torch.equal(timesteps, sigmas[:-1] * 1000)
    # exponential time shift of t: exp(mu) / (exp(mu) + 1/t - 1), here at the last unshifted step
    mu = calculate_shift(n)
    t = 1 / steps
    assert float(sigmas[steps - 1]) == pytest.approx(math.exp(mu) / (math.exp(mu) + 1 / t - 1), rel=1e-6)


def test_shift_raises_mid_sigmas_for_larger_images():
    small, _ = flux_sigmas(10, 1024)
    large, _ = flux_sigmas(10, 16384)
    assert bool((large[1:-1] > small[1:-1]).all())
