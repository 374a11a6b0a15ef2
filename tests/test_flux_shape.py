"""CPU checks of the FLUX-shaped transformer's configuration and small host-side formulas."""

import math

import torch

from hilberta_amd.flux_model import FluxShape, timestep_projection


def flux_dev_parameter_count(s: FluxShape = FluxShape()):
    """Parameters of diffusers' FluxTransformer2DModel at FLUX.1-dev's configuration, from the
    layer shapes: per double block two streams of AdaLN-zero (6C), QKV (3C), output (C) and MLP
    (4C, C) linears plus four 128-wide QK norms; per single block AdaLN (3C), QKV+MLP (3C+4C),
    output (C+4C -> C) and two norms; embedders, output norm and projection."""
    C, M = s.hidden, s.mlp_hidden
    lin = lambda o, i: o * i + o  # noqa: E731
    double = 2 * (lin(6 * C, C) + lin(3 * C, C) + lin(C, C) + lin(M, C) + lin(C, M)) + 4 * s.head_dim
    single = lin(3 * C, C) + lin(3 * C + M, C) + lin(C, C + M) + 2 * s.head_dim
    embed = (lin(C, s.in_channels) + lin(C, s.joint_attention_dim)
             + 2 * (lin(C, s.timestep_dim) + lin(C, C)) + lin(C, s.pooled_projection_dim) + lin(C, C)
             + lin(2 * C, C) + lin(s.in_channels, C))
    return s.num_layers * double + s.num_single_layers * single + embed


def test_flux_dev_shape():
    s = FluxShape()
    assert (s.hidden, s.mlp_hidden, s.blocks) == (3072, 12288, 57)
    # FLUX.1-dev's transformer has 11,901,408,320 parameters
    assert flux_dev_parameter_count(s) == 11_901_408_320


def test_timestep_projection_closed_form():
    t = torch.tensor([0.0, 500.0, 1000.0])
    emb = timestep_projection(t, 256)
    assert emb.shape == (3, 256)
    assert torch.equal(emb[0, :128], torch.ones(128)) and torch.equal(emb[0, 128:], torch.zeros(128))
    # column j of each half has frequency 10000^(-j/128): j = 0 -> the timestep itself
    assert math.isclose(float(emb[1, 0]), math.cos(500.0), abs_tol=1e-4)
    assert math.isclose(float(emb[2, 128 + 64]), math.sin(1000.0 * 10000 ** (-0.5)), abs_tol=1e-4)
