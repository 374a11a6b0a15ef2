"""CPU property mocks: host-side guards of the kernel entry points, no GPU touched.

Mirrors the reference's tests/test_sparse_kernel_contract.py and tests/test_paired_kernel_contract.py:
duck-typed tensors carry shape/stride/pointer/device; the HIP launchers are patched out.
"""

from types import SimpleNamespace
from unittest.mock import MagicMock, patch

import pytest
import torch

from hilberta_amd.paired_kernel import paired_attention
from hilberta_amd.sparse_kernel import _check_inputs, sparse_attention, validate_metadata


class TensorProperties:
    def __init__(self, shape, strides=None, dtype=torch.bfloat16, pointer=1_000_000, device="cuda:0",
                 requires_grad=False):
        self.shape = tuple(shape)
        self.ndim = len(shape)
        self.dtype = dtype
        self.device = torch.device(device)
        self.is_cuda = self.device.type == "cuda"
        self.requires_grad = requires_grad
        self.pointer = pointer
        if strides is None:
            strides, running = [], 1
            for size in reversed(shape):
                strides.insert(0, running)
                running *= size
        self.strides = tuple(strides)

    def stride(self, dim=None):
        return self.strides if dim is None else self.strides[dim]

    def data_ptr(self):
        return self.pointer

    def element_size(self):
        return 4 if self.dtype == torch.int32 else 2

    def is_contiguous(self):
        running = 1
        for size, stride in zip(reversed(self.shape), reversed(self.strides)):
            if size > 1 and stride != running:
                return False
            running *= size
        return True


SHAPE = (1, 2, 512, 128)
NATIVE = (131072, 128, 256, 1)


# ---------------------------------------------------------------- sparse_attention (unpaired)
@pytest.fixture
def sp():
    return SimpleNamespace(
        q=TensorProperties(SHAPE, NATIVE, pointer=1_000_000),
        k=TensorProperties(SHAPE, pointer=2_000_000),
        v=TensorProperties(SHAPE, NATIVE, pointer=3_000_000),
        ids=TensorProperties((6, 5), dtype=torch.int32, pointer=4_000_000),
        counts=TensorProperties((6,), dtype=torch.int32, pointer=5_000_000),
        out=TensorProperties(SHAPE, NATIVE, pointer=6_000_000),
    )


def check(sp, **changes):
    values = dict(q=sp.q, k=sp.k, v=sp.v, kv_indices=sp.ids, kv_counts=sp.counts, global_tokens=128,
                  block_size=64, out=sp.out)
    values.update(changes)
    return _check_inputs(**values)


def test_native_output_and_mixed_input_strides(sp):
    check(sp)
    check(sp, out=TensorProperties(SHAPE, pointer=6_000_000))


@pytest.mark.parametrize("source", ["q", "ids"])
def test_input_and_metadata_alias_rejected(sp, source):
    sp.out.pointer = getattr(sp, source).pointer
    with pytest.raises(ValueError, match="alias"):
        check(sp)


def test_partial_alias_rejected(sp):
    sp.out.pointer = sp.k.pointer + 1024
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
        q=TensorProperties(SHAPE, NATIVE, pointer=1_000_000),
        k=TensorProperties(SHAPE, pointer=2_000_000),
        v=TensorProperties(SHAPE, NATIVE, pointer=3_000_000),
        out=TensorProperties(SHAPE, NATIVE, pointer=7_000_000),
    )
    ns.meta = SimpleNamespace(
        tokens=512, global_tokens=128, key_block_size=64,
        kv_indices=TensorProperties((3, 5), dtype=torch.int32, pointer=4_000_000),
        kv_flags=TensorProperties((3, 5), dtype=torch.int32, pointer=5_000_000),
        kv_counts=TensorProperties((3,), dtype=torch.int32, pointer=6_000_000),
    )
    return ns


def pcall(pa, **kw):
    with patch("hilberta_amd.paired_kernel._paired_fwd", MagicMock()):
        return paired_attention(pa.q, pa.k, pa.v, pa.meta, out=pa.out, global_strategy="triton", **kw)


def test_paired_native_output(pa):
    assert pcall(pa) is pa.out


def test_paired_alias_rejected(pa):
    for src in (pa.q, pa.k, pa.v, pa.meta.kv_indices, pa.meta.kv_flags, pa.meta.kv_counts):
        pa.out.pointer = src.pointer
        with pytest.raises(ValueError, match="alias"):
            pcall(pa)
    pa.out.pointer = pa.k.pointer + 64
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
    pa.q.pointer = 1_000_002  # not 16-byte aligned
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
