"""Pins oracle/flux_ops.py (diffusers 0.36.0 RMSNorm / apply_rotary_emb / FluxPosEmbed restated)
against formulations that do not share its code: complex multiplication, closed forms, a float64
loop over the table definition, and group properties of the rotation."""

import math

import pytest
import torch

from oracle import flux_ops as F


def _complex_rotate(x, cos, sin):
    """(x[2i] + i x[2i+1]) * exp(i angle) with angle = atan2(sin, cos) of the even columns."""
    z = torch.view_as_complex(x.double().unflatten(-1, (-1, 2)).contiguous())
    angle = torch.atan2(sin[:, ::2].double(), cos[:, ::2].double())
    rot = torch.polar(torch.ones_like(angle), angle)[None, :, None, :]
    return torch.view_as_real(z * rot).flatten(-2)


def test_rotation_is_complex_multiplication():
    gen = torch.Generator().manual_seed(0)
    txt, img = F.flux_ids(4, 6)
    cos, sin = F.rotary_tables(torch.cat([txt, img]))
    x = torch.randn(2, 40, 3, 128, generator=gen)
    got = F.apply_rotary(x, cos, sin)            # fp32 in, fp32 out
    ref = _complex_rotate(x, cos, sin)
    assert torch.allclose(got.double(), ref, atol=2e-5, rtol=1e-5)
    # a sign or pair-order mistake in rotate_pairs would fail this on the odd or even columns
    assert (got[..., 1::2].double() - ref[..., 1::2]).abs().max() < 2e-5


def test_rotation_identity_composition_and_norm():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(1, 5, 2, 128, generator=gen, dtype=torch.float64).float()
    zero = torch.zeros(5, 3)
    c0, s0 = F.rotary_tables(zero)
    assert torch.equal(F.apply_rotary(x, c0, s0), x)
    a = torch.tensor([[0.0, 3.0, 5.0]] * 5)
    b = torch.tensor([[0.0, 4.0, 9.0]] * 5)
    ca, sa = F.rotary_tables(a)
    cb, sb = F.rotary_tables(b)
    cab, sab = F.rotary_tables(a + b)
    two = F.apply_rotary(F.apply_rotary(x, ca, sa), cb, sb)
    assert torch.allclose(two, F.apply_rotary(x, cab, sab), atol=1e-5)
    pair_norm = lambda t: t.unflatten(-1, (-1, 2)).norm(dim=-1)  # noqa: E731
    assert torch.allclose(pair_norm(F.apply_rotary(x, ca, sa)), pair_norm(x), atol=1e-5)


def test_rotary_tables_match_float64_loop():
    ids = torch.tensor([[0.0, 0.0, 0.0], [0.0, 1.0, 2.0], [0.0, 63.0, 17.0], [0.0, 127.0, 127.0],
                        [3.0, 5.0, 7.0]])
    cos, sin = F.rotary_tables(ids)
    lc, ls = F.rotary_tables_loop(ids)
    assert cos.shape == (5, 128) and cos.dtype == torch.float32
    assert torch.allclose(cos, lc, atol=1e-6, rtol=0) and torch.allclose(sin, ls, atol=1e-6, rtol=0)
    # column 0 of axis 1 (column 16) has frequency 1: the angle is the row coordinate itself
    assert math.isclose(float(cos[2, 16]), math.cos(63.0), abs_tol=1e-6)
    assert math.isclose(float(sin[3, 72]), math.sin(127.0), abs_tol=1e-6)


def test_flux_ids_layout():
    txt, img = F.flux_ids(3, 4)
    assert torch.equal(txt, torch.zeros(3, 3))
    assert img.shape == (16, 3)
    assert img[5].tolist() == [0.0, 1.0, 1.0] and img[7].tolist() == [0.0, 1.0, 3.0]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rms_norm_closed_forms(dtype):
    eps = 1e-6
    w = torch.linspace(0.5, 1.5, 128).to(dtype)
    const = torch.full((2, 128), -3.0, dtype=dtype)
    expect = (-1.0 / math.sqrt(1 + eps / 9.0)) * torch.ones(2, 128)
    got = F.rms_norm(const, w, eps)
    assert torch.equal(got, (expect.to(dtype) * w))
    one_hot = torch.zeros(1, 128, dtype=dtype)
    one_hot[0, 37] = 2.0
    got = F.rms_norm(one_hot, None, eps)
    assert got.dtype == dtype and int((got != 0).sum()) == 1
    assert math.isclose(float(got[0, 37]), math.sqrt(128 / (1 + 128 * eps / 4)), rel_tol=2 ** -7)


def test_rms_norm_float64_rows():
    gen = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 128, generator=gen) * 4).to(torch.bfloat16)
    w = (torch.rand(128, generator=gen) + 0.5).to(torch.bfloat16)
    xd = x.double()
    ref = (xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6)) * w.double()
    got = F.rms_norm(x, w).double()
    # two bf16 roundings (normalised value, weighted value): within 2 ulp relative
    assert ((got - ref).abs() <= 2 ** -7 * ref.abs() + 1e-30).all()


def test_qk_prep_sequence():
    gen = torch.Generator().manual_seed(4)
    txt, img = F.flux_ids(2, 3)
    cos, sin = F.rotary_tables(torch.cat([txt, img]))
    t = torch.randn(1, 2, 256, generator=gen).to(torch.bfloat16)
    i = torch.randn(1, 9, 256, generator=gen).to(torch.bfloat16)
    wt = torch.rand(128, generator=gen).to(torch.bfloat16)
    wi = torch.rand(128, generator=gen).to(torch.bfloat16)
    out = F.qk_prep(t, i, heads=2, weight_text=wt, weight_image=wi, cos=cos, sin=sin)
    assert out.shape == (1, 11, 2, 128)
    # text rows have position 0 (identity rotation) and the text weight
    assert torch.equal(out[:, :2], F.rms_norm(t.unflatten(-1, (2, 128)), wt))
    mid = F.rms_norm(i.unflatten(-1, (2, 128)), wi)
    assert torch.equal(out[:, 2:], F.apply_rotary(mid, cos[2:], sin[2:]))
    plain = F.qk_prep(t, i, heads=2, normalize=False)
    assert torch.equal(plain, torch.cat([t, i], 1).unflatten(-1, (2, 128)))
