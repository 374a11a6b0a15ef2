"""GPU parity of the fused gated-residual + AdaLN kernel (csrc/adaln.hip) against the torch
sequence the FLUX blocks run (diffusers 0.36.0): r = addcmul(x, gate, y); n = layer_norm(r);
out = addcmul(shift, n, 1 + scale) -- on the same device, and against float64 arithmetic.

Tolerance (a floating-point kernel): the residual r rounds the same fp32 value as torch's addcmul
(bitwise for >= 99.9 % of the elements, else one unit in the last place); the LayerNorm
statistics are reduced in another order, so the normalised value may round to its neighbour:
>= 99.9 % of the outputs are bitwise equal and every one is within
2^-6 * (|shift| + |n| * |1 + scale|) of the torch result.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import say

pytestmark = pytest.mark.gpu


def _torch_sequence(x, shift, scale, y=None, gate=None, eps=1e-6):
    r = x if y is None else torch.addcmul(x, gate[:, None], y)
    n = F.layer_norm(r, (x.shape[-1],), eps=eps)
    return r, n, torch.addcmul(shift[:, None], n, (1 + scale)[:, None])


def _check(got, ref, n, shift, scale, what):
    bound = 2 ** -6 * (shift[:, None].float().abs() + n.float().abs() * (1 + scale[:, None]).float().abs())
    diff = (got.float() - ref.float()).abs()
    equal = float((got == ref).float().mean())
    say(f"{what}: bitwise-equal fraction {equal:.6f}, max abs diff {float(diff.max()):.3e}")
    assert equal >= 0.999, what
    assert bool((diff <= bound + 1e-6).all()), what


@pytest.mark.parametrize("dtype,hidden,B,R", [(torch.bfloat16, 3072, 1, 16384), (torch.bfloat16, 512, 2, 700),
                                              (torch.float16, 3072, 2, 513), (torch.bfloat16, 1536, 1, 64)])
def test_residual_and_modulation(hip_device, dtype, hidden, B, R):
    from hilberta_amd.flux_norm import adaln_modulate

    gen = torch.Generator("cpu").manual_seed(hidden + R)
    x = (torch.randn(B, R, hidden, generator=gen) * 2 + 0.5).to(dtype).to(hip_device)
    y = torch.randn(B, R, hidden, generator=gen).to(dtype).to(hip_device)
    mod = (torch.randn(B, 6 * hidden, generator=gen) * 0.5).to(dtype).to(hip_device)
    shift, scale, gate = mod[:, :hidden], mod[:, 2 * hidden:3 * hidden], mod[:, 5 * hidden:]
    say(f"case adaln {dtype} hidden {hidden} B={B} rows {R}")
    r_ref, n_ref, out_ref = _torch_sequence(x, shift, scale, y, gate)
    x_new = torch.empty_like(x)
    out = adaln_modulate(x, shift, scale, y=y, gate=gate, x_out=x_new)
    torch.cuda.synchronize()
    assert float((x_new == r_ref).float().mean()) >= 0.999
    ulp = 2.0 ** (torch.floor(torch.log2(r_ref.float().abs().clamp_min(1e-30))) - (7 if dtype == torch.bfloat16 else 10))
    assert bool(((x_new.float() - r_ref.float()).abs() <= ulp).all())
    # the rest of the comparison starts from the kernel's own residual
    _, n_ref, out_ref = _torch_sequence(x_new, shift, scale)
    _check(out, out_ref, n_ref, shift, scale, "modulated")
    # float64: LayerNorm of the stored residual, modulated, against the kernel output
    r64 = x_new.double()
    n64 = (r64 - r64.mean(-1, keepdim=True)) / torch.sqrt(r64.var(-1, unbiased=False, keepdim=True) + 1e-6)
    o64 = shift[:, None].double() + n64 * (1 + scale[:, None].double())
    assert float((out.double() - o64).abs().mean()) < 2e-2 * float(o64.abs().mean())


def test_in_place_residual_and_strided_rows(hip_device):
    """x_out aliasing x (in-place residual) and row ranges of one [B, N, C] tensor, as the blocks
    use them (image rows T.. and text rows 0..T written into one joint buffer)."""
    from hilberta_amd.flux_norm import adaln_modulate

    gen = torch.Generator("cpu").manual_seed(5)
    C, T, n = 3072, 512, 1024
    x = torch.randn(1, n, C, generator=gen).to(torch.bfloat16).to(hip_device)
    y = torch.randn(1, n, C, generator=gen).to(torch.bfloat16).to(hip_device)
    mod = (torch.randn(1, 3 * C, generator=gen) * 0.3).to(torch.bfloat16).to(hip_device)
    shift, scale, gate = mod.chunk(3, dim=1)
    joint = torch.zeros(1, T + n, C, dtype=torch.bfloat16, device=hip_device)
    joint_n = torch.zeros_like(joint)
    say("case adaln in place + joint rows")
    a = adaln_modulate(x.clone(), shift, scale, y=y, gate=gate, x_out=joint[:, T:], out=joint_n[:, T:])
    x2 = x.clone()
    b = adaln_modulate(x2, shift, scale, y=y, gate=gate, x_out=x2)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(joint[:, T:], x2)
    assert bool((joint[:, :T] == 0).all()) and bool((joint_n[:, :T] == 0).all())
    c = adaln_modulate(x2, shift, scale)          # no residual update
    assert torch.equal(c, b)


def test_argument_errors(hip_device):
    from hilberta_amd.flux_norm import adaln_modulate

    x = torch.zeros(1, 4, 3072, dtype=torch.bfloat16, device=hip_device)
    m = torch.zeros(1, 3072, dtype=torch.bfloat16, device=hip_device)
    with pytest.raises(ValueError):
        adaln_modulate(x, m, m, y=x)
    with pytest.raises(ValueError):
        adaln_modulate(x, m, m, x_out=x)
    with pytest.raises(ValueError):
        adaln_modulate(x[..., :1000], m[:, :1000], m[:, :1000])
