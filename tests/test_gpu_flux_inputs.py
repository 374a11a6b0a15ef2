"""GPU parity of the fused QK RMSNorm + rotary + [text; image] BNHD kernel (csrc/qk_prep.hip)
against the diffusers 0.36.0 formulas restated in oracle/flux_ops.py, evaluated with torch on the
same device in fp32.

Tolerances (a floating-point kernel):
  * without RMSNorm (rotation only, or plain concatenation) the kernel rounds exactly as the
    unfused fp32 formula: bitwise equal;
  * with RMSNorm the sum of squares is reduced in another order and rsqrt may differ in the last
    fp32 bit, so a normalised value can round to the neighbouring bf16/fp16 value: at least
    99.9% of the elements are bitwise equal, and every element is within 2^-6 * (|y_2i| + |y_2i+1|)
    of the reference, y being the oracle's normalised pair before the rotation (one unit in the
    last place of each input of the rotation plus one of its output).
"""

import pytest
import torch

from oracle import flux_ops as F
from tests.helpers import say

pytestmark = pytest.mark.gpu

D = 128


def _inputs(device, B, T, n, heads, dtype, seed, scale=3.0):
    gen = torch.Generator("cpu").manual_seed(seed)
    t = (torch.randn(B, T, heads * D, generator=gen) * scale).to(dtype).to(device)
    i = (torch.randn(B, n, heads * D, generator=gen) * scale).to(dtype).to(device)
    wt = (torch.rand(D, generator=gen) * 1.5 + 0.25).to(dtype).to(device)
    wi = (torch.rand(D, generator=gen) * 1.5 + 0.25).to(dtype).to(device)
    return t, i, wt, wi


def _tables(device, T, grid, permute_seed=None):
    txt, img = F.flux_ids(T, grid)
    if permute_seed is not None:
        img = img[torch.randperm(len(img), generator=torch.Generator().manual_seed(permute_seed))]
    cos, sin = F.rotary_tables(torch.cat([txt, img]).to(device))
    return cos.contiguous(), sin.contiguous()


def _check_normed(got, t, i, heads, wt, wi, cos, sin, what):
    ref = F.qk_prep(t, i, heads=heads, weight_text=wt, weight_image=wi, cos=cos, sin=sin)
    y = F.qk_prep(t, i, heads=heads, weight_text=wt, weight_image=wi).float()
    pair = y.unflatten(-1, (-1, 2)).abs().sum(-1).repeat_interleave(2, -1)
    diff = (got.float() - ref.float()).abs()
    equal = float((got == ref).float().mean())
    worst = float((diff - 2 ** -6 * pair).max())
    say(f"{what}: bitwise-equal fraction {equal:.6f}, max abs diff {float(diff.max()):.3e}")
    assert equal >= 0.999, what
    assert worst <= 0, what


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rotation_only_and_concat_bitwise(hip_device, dtype):
    from hilberta_amd.flux_inputs import qk_prep

    heads, T, grid = 3, 40, 16
    t, i, _, _ = _inputs(hip_device, 2, T, grid * grid, heads, dtype, seed=1)
    cos, sin = _tables(hip_device, T, grid, permute_seed=2)
    say(f"case qk_prep rotation only {dtype}")
    got = qk_prep(t, i, heads=heads, normalize=False, cos=cos, sin=sin)
    ref = F.qk_prep(t, i, heads=heads, normalize=False, cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    say(f"case qk_prep concatenation {dtype}")
    got = qk_prep(t, i, heads=heads, normalize=False)
    assert torch.equal(got, torch.cat([t, i], 1).unflatten(-1, (heads, D)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_norm_rotation_small(hip_device, dtype):
    from hilberta_amd.flux_inputs import qk_prep

    heads, T, grid = 4, 24, 12
    t, i, wt, wi = _inputs(hip_device, 2, T, grid * grid, heads, dtype, seed=3)
    cos, sin = _tables(hip_device, T, grid)
    say(f"case qk_prep norm+rotation {dtype}")
    got = qk_prep(t, i, heads=heads, weight_text=wt, weight_image=wi, cos=cos, sin=sin)
    torch.cuda.synchronize()
    _check_normed(got, t, i, heads, wt, wi, cos, sin, f"small {dtype}")
    say(f"case qk_prep norm without weights {dtype}")
    got = qk_prep(t, i, heads=heads)
    ref = F.qk_prep(t, i, heads=heads)
    assert float((got == ref).float().mean()) >= 0.999
    assert float(((got.float() - ref.float()).abs() - 2 ** -7 * ref.float().abs()).max()) <= 0


def test_fused_projection_slices_2048(hip_device):
    """FLUX 2048 px shape: Q/K/V column slices of one fused [B, N, 3*3072] projection, the text
    rows from a second tensor, output into preallocated BNHD buffers, Hilbert-permuted ids."""
    from hilberta_amd.flux_inputs import qk_prep

    heads, T, grid = 24, 512, 128
    gen = torch.Generator("cpu").manual_seed(5)
    img = (torch.randn(1, grid * grid, 3 * heads * D, generator=gen)).to(torch.bfloat16).to(hip_device)
    txt = (torch.randn(1, T, 3 * heads * D, generator=gen)).to(torch.bfloat16).to(hip_device)
    wq = [(torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16).to(hip_device) for _ in range(4)]
    cos, sin = _tables(hip_device, T, grid, permute_seed=6)
    N = T + grid * grid
    out = torch.empty(3, 1, N, heads, D, dtype=torch.bfloat16, device=hip_device)
    say("case qk_prep 2048 fused slices")
    W = heads * D
    for j in range(3):
        kw = dict(weight_text=wq[2 * j], weight_image=wq[2 * j + 1], cos=cos, sin=sin) if j < 2 else \
            dict(normalize=False)
        qk_prep(txt[..., j * W:(j + 1) * W], img[..., j * W:(j + 1) * W], heads=heads, out=out[j], **kw)
    torch.cuda.synchronize()
    for j in range(2):
        _check_normed(out[j], txt[..., j * W:(j + 1) * W], img[..., j * W:(j + 1) * W], heads,
                      wq[2 * j], wq[2 * j + 1], cos, sin, f"2048 slice {j}")
    assert torch.equal(out[2], torch.cat([txt[..., 2 * W:], img[..., 2 * W:]], 1).unflatten(-1, (heads, D)))


def test_single_source_rows(hip_device):
    """Single-stream blocks: text and image are row ranges of one [B, N, C] tensor, one weight."""
    from hilberta_amd.flux_inputs import qk_prep

    heads, T, grid = 24, 512, 64
    gen = torch.Generator("cpu").manual_seed(7)
    N = T + grid * grid
    x = torch.randn(2, N, 4 * heads * D, generator=gen).to(torch.bfloat16).to(hip_device)
    w = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16).to(hip_device)
    cos, sin = _tables(hip_device, T, grid, permute_seed=8)
    q = x[..., heads * D:2 * heads * D]
    say("case qk_prep single source 1024 B=2")
    got = qk_prep(q[:, :T], q[:, T:], heads=heads, weight_text=w, weight_image=w, cos=cos, sin=sin)
    torch.cuda.synchronize()
    _check_normed(got, q[:, :T], q[:, T:], heads, w, w, cos, sin, "single source")


def test_argument_errors(hip_device):
    from hilberta_amd.flux_inputs import qk_prep

    t, i, wt, wi = _inputs(hip_device, 1, 8, 16, 2, torch.bfloat16, seed=9)
    cos, sin = _tables(hip_device, 8, 4)
    with pytest.raises(ValueError):
        qk_prep(t, i, heads=3)
    with pytest.raises(ValueError):
        qk_prep(t, i, heads=2, cos=cos)
    with pytest.raises(ValueError):
        qk_prep(t, i, heads=2, cos=cos[:-1], sin=sin[:-1])
    with pytest.raises(ValueError):
        qk_prep(t, i, heads=2, normalize=False, weight_text=wt)
    with pytest.raises(ValueError):
        qk_prep(t.float(), i.float(), heads=2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pair_launch_equals_two_single_launches(hip_device, dtype):
    """planes=2 (Q and K from one fused projection in one launch) gives the same bits as two
    single-plane launches, and matches the formulas within the tolerance above."""
    from hilberta_amd.flux_inputs import qk_prep, qk_prep_pair

    heads, T, grid = 24, 512, 64
    W = heads * D
    gen = torch.Generator("cpu").manual_seed(11)
    N = T + grid * grid
    qkv = torch.randn(2, N, 3 * W, generator=gen).to(dtype).to(hip_device)
    w = [(torch.rand(D, generator=gen) + 0.5).to(dtype).to(hip_device) for _ in range(4)]
    cos, sin = _tables(hip_device, T, grid, permute_seed=12)
    say(f"case qk_prep_pair {dtype}")
    qk = qk_prep_pair(qkv[:, :T, :2 * W], qkv[:, T:, :2 * W], heads=heads,
                      weights=((w[0], w[1]), (w[2], w[3])), cos=cos, sin=sin)
    q = qk_prep(qkv[:, :T, :W], qkv[:, T:, :W], heads=heads, weight_text=w[0], weight_image=w[1],
                cos=cos, sin=sin)
    k = qk_prep(qkv[:, :T, W:2 * W], qkv[:, T:, W:2 * W], heads=heads, weight_text=w[2],
                weight_image=w[3], cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert torch.equal(qk[0], q) and torch.equal(qk[1], k)
    _check_normed(qk[1], qkv[:, :T, W:2 * W], qkv[:, T:, W:2 * W], heads, w[2], w[3], cos, sin,
                  f"pair plane 1 {dtype}")
