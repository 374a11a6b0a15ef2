"""CPU property mocks: host-side guards of the kernel entry points, no GPU touched.

Mirrors the reference's tests/test_sparse_kernel_contract.py and tests/test_paired_kernel_contract.py:
host views (HostView) stand in for device tensors; the HIP launchers are patched out.
"""

from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Optional
from unittest.mock import MagicMock, patch

import pytest
import torch

from hilberta_amd.paired_kernel import paired_attention
from hilberta_amd.sparse_kernel import _check_inputs, sparse_attention, validate_metadata


@dataclass
class HostView:
    """A device tensor as the host-side checks see it, with no device memory behind it: sizes,
    element strides, dtype, device, autograd flag and the base address (for alias checks).  The
    stride arithmetic is delegated to a meta tensor of the same geometry."""

    shape: tuple
    strides: Optional[tuple] = None
    dtype: torch.dtype = torch.bfloat16
    address: int = 1 << 20
    device: torch.device = field(default_factory=lambda: torch.device("cuda", 0))
    requires_grad: bool = False

    def __post_init__(self):
        if self.strides is None:
            self.strides = torch.empty(self.shape, device="meta").stride()

    def _meta(self):
        return torch.empty_strided(self.shape, self.strides, dtype=self.dtype, device="meta")

    ndim = property(lambda self: len(self.shape))
    is_cuda = property(lambda self: self.device.type == "cuda")

    def stride(self, dim=None):
        return tuple(self.strides) if dim is None else self.strides[dim]

    def data_ptr(self):
        return self.address

    def element_size(self):
        return self._meta().element_size()

    def is_contiguous(self):
        return self._meta().is_contiguous()


SHAPE = (1, 2, 512, 128)
NATIVE = (131072, 128, 256, 1)


# ---------------------------------------------------------------- sparse_attention (unpaired)
@pytest.fixture
def sp():
    return SimpleNamespace(
        q=HostView(SHAPE, NATIVE, address=1_000_000),
        k=HostView(SHAPE, address=2_000_000),
        v=HostView(SHAPE, NATIVE, address=3_000_000),
        ids=HostView((6, 5), dtype=torch.int32, address=4_000_000),
        counts=HostView((6,), dtype=torch.int32, address=5_000_000),
        out=HostView(SHAPE, NATIVE, address=6_000_000),
    )


def check(sp, **changes):
    values = dict(q=sp.q, k=sp.k, v=sp.v, kv_indices=sp.ids, kv_counts=sp.counts, global_tokens=128,
                  block_size=64, out=sp.out)
    values.update(changes)
    return _check_inputs(**values)


def test_native_output_and_mixed_input_strides(sp):
    check(sp)
    check(sp, out=HostView(SHAPE, address=6_000_000))


@pytest.mark.parametrize("source", ["q", "ids"])
def test_input_and_metadata_alias_rejected(sp, source):
    sp.out.address = getattr(sp, source).address
    with pytest.raises(ValueError, match="alias"):
        check(sp)


def test_partial_alias_rejected(sp):
    sp.out.address = sp.k.address + 1024
    with pytest.raises(ValueError, match="alias"):
        check(sp)


def test_overlapping_and_zero_stride_output_rejected(sp):
    sp.out.strides = (131072, 128, 128, 1)
    with pytest.raises(ValueError, match="non-overlapping"):
        check(sp)
    sp.out.strides = (0, 128, 256, 1)
    with pytest.raises(ValueError, match="positive"):
        check(sp)


def test_gradients_rejected(sp):
    sp.q.requires_grad = True
    with torch.enable_grad(), pytest.raises(ValueError, match="inference-only"):
        check(sp)
    with torch.no_grad():
        check(sp)
    sp.q.requires_grad = False
    sp.out.requires_grad = True
    with torch.enable_grad(), pytest.raises(ValueError, match="gradients"):
        check(sp)


@pytest.mark.parametrize("value", [128.0, True])
def test_noninteger_global_rejected(sp, value):
    with pytest.raises(TypeError):
        check(sp, global_tokens=value)


def test_empty_batch_rejected(sp):
    sp.q.shape = sp.k.shape = sp.v.shape = (0, 2, 512, 128)
    with pytest.raises(ValueError, match="nonempty"):
        check(sp, out=None)


def test_tensor_scale_and_float_tuning_rejected(sp):
    with pytest.raises(TypeError, match="never a tensor"):
        sparse_attention(sp.q, sp.k, sp.v, sp.ids, sp.counts, global_tokens=128, scale=torch.tensor(1.0))
    with pytest.raises(TypeError, match="tuning"):
        sparse_attention(sp.q, sp.k, sp.v, sp.ids, sp.counts, global_tokens=128, num_warps=4.0)


def test_wrong_device_rejected(sp):
    sp.v.device = torch.device("cuda:1")
    with pytest.raises(ValueError, match="one CUDA"):
        check(sp)


def test_sparse_launch_reaches_hip_launcher(sp):
    with patch("hilberta_amd.sparse_kernel._block_sparse_fwd", MagicMock()) as launcher:
        res = sparse_attention(sp.q, sp.k, sp.v, sp.ids, sp.counts, global_tokens=128, out=sp.out)
    assert res is sp.out
    launcher.assert_called_once()


# ---------------------------------------------------------------- paired_attention
@pytest.fixture
def pa():
    ns = SimpleNamespace(
        q=HostView(SHAPE, NATIVE, address=1_000_000),
        k=HostView(SHAPE, address=2_000_000),
        v=HostView(SHAPE, NATIVE, address=3_000_000),
        out=HostView(SHAPE, NATIVE, address=7_000_000),
    )
    ns.meta = SimpleNamespace(
        tokens=512, global_tokens=128, key_block_size=64,
        kv_indices=HostView((3, 5), dtype=torch.int32, address=4_000_000),
        kv_flags=HostView((3, 5), dtype=torch.int32, address=5_000_000),
        kv_counts=HostView((3,), dtype=torch.int32, address=6_000_000),
    )
    return ns


def pcall(pa, **kw):
    with patch("hilberta_amd.paired_kernel._paired_fwd", MagicMock()):
        return paired_attention(pa.q, pa.k, pa.v, pa.meta, out=pa.out, global_strategy="triton", **kw)


def test_paired_native_output(pa):
    assert pcall(pa) is pa.out


def test_paired_alias_rejected(pa):
    for src in (pa.q, pa.k, pa.v, pa.meta.kv_indices, pa.meta.kv_flags, pa.meta.kv_counts):
        pa.out.address = src.address
        with pytest.raises(ValueError, match="alias"):
            pcall(pa)
    pa.out.address = pa.k.address + 64
    with pytest.raises(ValueError, match="alias"):
        pcall(pa)


def test_paired_overlap_and_zero_stride(pa):
    for strides in ((131072, 128, 128, 1), (0, 128, 256, 1)):
        pa.out.strides = strides
        with pytest.raises(ValueError, match="non-overlapping"):
            pcall(pa)


def test_paired_grad_and_scale_and_tuning(pa):
    pa.q.requires_grad = True
    with torch.enable_grad(), pytest.raises(ValueError, match="Inference"):
        pcall(pa)
    with torch.no_grad():
        pcall(pa)
    pa.q.requires_grad = False
    pa.out.requires_grad = True
    with torch.enable_grad(), pytest.raises(ValueError, match="gradients"):
        pcall(pa)
    pa.out.requires_grad = False
    with pytest.raises(TypeError, match="never a tensor"):
        pcall(pa, scale=torch.tensor(1.0))
    for value in (4.0, True):
        with pytest.raises(TypeError, match="Integer"):
            pcall(pa, num_warps=value)


def test_paired_metadata_checks(pa):
    pa.meta.kv_flags.device = torch.device("cuda:1")
    with pytest.raises(ValueError, match="CUDA"):
        pcall(pa)
    pa.meta.kv_flags.device = torch.device("cuda:0")
    pa.meta.kv_flags.shape = (3, 4)
    with pytest.raises(ValueError, match="shape"):
        pcall(pa)
    pa.meta.kv_flags.shape = (3, 5)
    pa.meta.global_tokens = 64
    with pytest.raises(ValueError, match="alignment"):
        pcall(pa)
    pa.meta.global_tokens = 128
    pa.k.strides = (131072, -128, 256, 1)
    with pytest.raises(ValueError, match="Positive"):
        pcall(pa)


def test_vector_alignment_required(pa):
    pa.q.address = 1_000_002  # not 16-byte aligned
    with pytest.raises(ValueError, match="16-byte"):
        pcall(pa)


def test_lse_buffer_checked(pa):
    with pytest.raises(ValueError, match="lse"):
        pcall(pa, lse=torch.empty(1, 2, 512))  # CPU tensor: wrong device


# ---------------------------------------------------------------- validate_metadata (host logic)
def test_validate_metadata_messages():
    ids = torch.tensor([[0, 1], [0, 2]], dtype=torch.int32)
    counts = torch.tensor([2, 2], dtype=torch.int32)
    info = validate_metadata(ids, counts, tokens=192, global_tokens=64)
    assert info["total_directed_entries"] == 64 * 192 + 4 * 4096
    with pytest.raises(ValueError, match="duplicate"):
        validate_metadata(torch.tensor([[0, 0], [0, 2]], dtype=torch.int32), counts, tokens=192,
                          global_tokens=64)
    with pytest.raises(ValueError, match="global-prefix"):
        validate_metadata(torch.tensor([[1, 2], [0, 2]], dtype=torch.int32), counts, tokens=192,
                          global_tokens=64)
    with pytest.raises(ValueError, match="Invalid K/V count"):
        validate_metadata(ids, torch.tensor([3, 2], dtype=torch.int32), tokens=192, global_tokens=64)
    with pytest.raises(TypeError):
        validate_metadata(ids.long(), counts, tokens=192, global_tokens=64)
    with pytest.raises(ValueError, match="Out-of-range"):
        validate_metadata(torch.tensor([[0, 3], [0, 2]], dtype=torch.int32), counts, tokens=192,
                          global_tokens=64)
    # padding beyond the count may hold anything
    validate_metadata(torch.tensor([[0, 1], [0, -1]], dtype=torch.int32),
                      torch.tensor([2, 1], dtype=torch.int32), tokens=192, global_tokens=64)
