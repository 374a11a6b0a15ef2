"""HilbertA inference attention path for AMD Instinct MI355X (gfx950).

Composite-Hilbert token layout, sliding tiles and reciprocal block bridges (wenboluu/hilberta),
rebuilt on hand-written HIP kernels behind a C ABI (include/hilberta_hip.h):

  layout            Hilbert permute / unpermute of token rows (HIP gather)
  geometry / plan / bridge_k / paired_metadata
                    block tables built on the GPU, bit-exact with the reference
  paired_kernel / sparse_kernel
                    block-sparse flash-attention forward (bf16/fp16 MFMA, persistent)
  flux_inputs / flux_norm
                    FLUX attention inputs (RMSNorm + rotary + [text; image] layout) and the
                    gated-residual AdaLN pass, one HIP kernel each
  flux_model / sampling_layout
                    a FLUX-shaped denoiser step on these kernels and the sampling-scope layout
  ops               the entry points as torch custom ops (torch.ops.hilberta_hip.*), with fake
                    implementations for tracing

The modules keep the reference package's call surface.  There is no CPU fallback: the HIP library
(python -m hilberta_amd.build) and a GPU are required for every computation.
"""

from . import ops
from .bridge_k import bridge_k_plan

__version__ = "0.1.0"

__all__ = ["bridge_k_plan"]
