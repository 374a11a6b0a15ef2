"""FLUX.1-dev-shaped denoiser transformer (random init) whose joint attention runs on the HIP path.

The reference accelerates diffusers' FluxTransformer2DModel by replacing one operation per block
(hilberta/flux_adapter.py:255-340, PersistentFluxProcessor) and by holding the image tokens in the
persistent Hilbert layout for the whole transformer call (flux_adapter.py:149-252).  diffusers is
not available here, so this module restates that transformer's structure (diffusers 0.36.0
FluxTransformer2DModel with FLUX.1-dev's configuration) with random weights, to time one denoiser
step at the real shapes:

  * embedders: x (64 -> 3072), context (4096 -> 3072), timestep / guidance / pooled-text MLPs;
  * 19 double-stream blocks: AdaLN-zero modulation per stream, QKV projections, per-head QK
    RMSNorm, 3-axis RoPE (theta 10000, axes 16/56/56), joint [text; image] attention, output
    projections, gated residuals, GELU(tanh) MLPs with ratio 4;
  * 38 single-stream blocks over [text; image]: modulation, one fused QKV + MLP projection,
    attention, concatenated output projection;
  * AdaLN-continuous output norm and the 3072 -> 64 projection.

Q and K are prepared by one HIP pass (flux_inputs.qk_prep_pair: RMSNorm + rotation +
[text; image] concatenation straight into the [B, N, H, D] storage the kernels read), V is read in
place from the joint QKV projection, and every gated residual add is fused with the next AdaLN
modulation (flux_norm.adaln_modulate).  Two attention modes:

  * ``NativeAttention``: raster token order and dense attention on the same GPU (torch's
    scaled_dot_product_attention, flash / memory-efficient backends) -- the "full attention"
    comparison of the reference's denoiser rows;
  * ``PersistentAttention``: image tokens and ids gathered into the plan's order once at entry,
    block ``i`` of the 57 (double blocks first) attends with the plan's phase ``i % 4``
    (flux_adapter.py:421, :269), the prediction gathered back to raster order once at exit
    (flux_adapter.py:243).  Backends: ``paired`` (paired_kernel.paired_attention), ``sparse``
    (sparse_kernel.sparse_attention on unpaired tables) and ``sdpa_reference`` (dense-mask SDPA,
    a correctness reference as at flux_adapter.py:299-306).

Weights and activations are bf16; there is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .flux_inputs import qk_prep_pair, rotary_tables
from .flux_norm import adaln_modulate
from .layout import index_select_rows


@dataclass(frozen=True)
class FluxShape:
    """FLUX.1-dev transformer hyper-parameters (diffusers FluxTransformer2DModel config)."""

    num_layers: int = 19
    num_single_layers: int = 38
    heads: int = 24
    head_dim: int = 128
    mlp_ratio: float = 4.0
    in_channels: int = 64
    joint_attention_dim: int = 4096
    pooled_projection_dim: int = 768
    timestep_dim: int = 256
    guidance_embeds: bool = True
    eps: float = 1e-6

    @property
    def hidden(self):
        return self.heads * self.head_dim

    @property
    def mlp_hidden(self):
        return int(self.hidden * self.mlp_ratio)

    @property
    def blocks(self):
        return self.num_layers + self.num_single_layers


class _Init:
    """Seeded random weights on the device: N(0, 1/fan_in) matrices, N(0, 0.02^2) biases, norm
    weights around 1."""

    def __init__(self, device, dtype, seed):
        self.device, self.dtype = device, dtype
        self.gen = torch.Generator(device=device)
        self.gen.manual_seed(seed)

    def linear(self, fan_out, fan_in, std=None, *, out_features=None, in_features=None, bias=True):
        """(weight [out_features, in_features], bias) with N(0, std^2), std defaulting to
        fan_in^-0.5; the feature counts default to fan_out / fan_in (a column block of a larger
        layer passes its own)."""
        shape = (out_features or fan_out, in_features or fan_in)
        w = torch.empty(shape, device=self.device, dtype=self.dtype)
        w.normal_(0.0, std if std is not None else fan_in**-0.5, generator=self.gen)
        if not bias:
            return w, None
        b = torch.empty(shape[0], device=self.device, dtype=self.dtype).normal_(0.0, 0.02, generator=self.gen)
        return w, b

    def norm(self, dim):
        w = torch.empty(dim, device=self.device, dtype=self.dtype)
        return w.normal_(1.0, 0.1, generator=self.gen)

    def mlp(self, fan_in, hidden):
        return self.linear(hidden, fan_in), self.linear(hidden, hidden)


def timestep_projection(t, dim=256):
    """diffusers get_timestep_embedding(flip_sin_to_cos=True, downscale_freq_shift=0): [cos | sin]
    of t * 10000^(-j/half)."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    angles = t[:, None].float() * freqs[None, :]
    return torch.cat([angles.cos(), angles.sin()], dim=-1)


def _mlp(x, layers):
    (w1, b1), (w2, b2) = layers
    return F.linear(F.silu(F.linear(x, w1, b1)), w2, b2)


class NativeAttention:
    """Dense attention in raster order on the same GPU (the full-attention comparison)."""

    layout = None

    def __call__(self, layer, q, k, v, out):
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out.copy_(F.scaled_dot_product_attention(q, k, v))


class PersistentAttention:
    """Persistent plan layout and per-block phase tables (flux_adapter.py:26-147, :255-340).

    ``plan`` is either a ``bridge_k.DevicePlan`` (paired tables built on the GPU; ``paired`` only)
    or an ``plan.AttentionPlan`` (from ``bridge_k_plan`` / ``build_plan``), whose tables are moved
    to ``device`` once here and paired on the GPU.
    """

    BACKENDS = ("paired", "sparse", "sdpa_reference")

    def __init__(self, plan, device, backend="paired", kernel_options=None):
        from .bridge_k import DevicePlan
        from .paired_metadata import pair_metadata_device
        from .sparse_kernel import validate_metadata

        if backend not in self.BACKENDS:
            raise ValueError("backend must be paired/sparse/sdpa_reference")
        self.backend = backend
        self.kernel_options = dict(kernel_options or {})
        self.global_tokens = plan.global_tokens
        self.total_tokens = plan.total_tokens
        self.calls = 0
        if isinstance(plan, DevicePlan):
            if backend != "paired":
                raise ValueError("a DevicePlan carries paired tables only")
            self.order = plan.layout.image_order.to(device)
            self.inverse = plan.layout.inverse_image_order.to(device)
            self.paired = list(plan.phases)
            self.tables = None
            self.plan = None
        else:
            self.order = plan.image_order.to(device=device, dtype=torch.int64)
            self.inverse = plan.inverse_image_order.to(device=device, dtype=torch.int64)
            cpu = [(p.kv_indices.cpu(), p.kv_counts.cpu()) for p in plan.phases]
            for ids, counts in cpu:   # validated once, on the CPU, before they are cached on the GPU
                validate_metadata(ids, counts, tokens=plan.total_tokens, global_tokens=plan.global_tokens,
                                  block_size=plan.block_size)
            if backend == "paired" and (plan.total_tokens % 128 or plan.global_tokens % 128):
                raise ValueError("Paired queries require N/global aligned to 128; KV must be 64/128")
            self.tables = [(ids.to(device), counts.to(device)) for ids, counts in cpu]
            self.paired = [
                pair_metadata_device(ids, counts, tokens=plan.total_tokens,
                                     global_tokens=plan.global_tokens, device=device, validated=True)
                for ids, counts in self.tables
            ] if backend == "paired" else None
            self.plan = plan
            self.block_size = plan.block_size
        self.masks = {}

    layout = property(lambda self: self)

    def __call__(self, layer, q, k, v, out):
        phase = layer % 4
        self.calls += 1
        if self.backend == "paired":
            from .paired_kernel import paired_attention

            paired_attention(q, k, v, self.paired[phase], out=out, **self.kernel_options)
        elif self.backend == "sparse":
            from .sparse_kernel import sparse_attention

            ids, counts = self.tables[phase]
            sparse_attention(q, k, v, ids, counts, global_tokens=self.global_tokens,
                             block_size=self.block_size, out=out, **self.kernel_options)
        else:
            if phase not in self.masks:
                self.masks[phase] = self.plan.dense_mask(phase, q.device)
            out.copy_(F.scaled_dot_product_attention(q, k, v, attn_mask=self.masks[phase]))


def _linear_into(x, weight, bias, out):
    """out[b] = x[b] @ weight^T + bias for every batch row, written in place (out may be a row
    range of a larger buffer: one GEMM per batch element writes straight into it)."""
    for b in range(x.shape[0]):
        torch.addmm(bias, x[b], weight.t(), out=out[b])


def _gelu_linear(x, weight, bias):
    """GELU(tanh)(x @ weight^T + bias) with the activation in the GEMM epilogue."""
    flat = x.reshape(-1, x.shape[-1])
    return torch._addmm_activation(bias, flat, weight.t(), use_gelu=True).view(*x.shape[:-1], -1)


def _joint_ranges(T, N):
    """Row ranges [text | image] of a joint sequence of T text and N - T image tokens.

    The single blocks' GEMMs run once per range: hipBLASLt takes a joint 16896-row GEMM at
    1.05-1.2 PFLOP/s but the 16384 image rows alone at 1.5-1.8 (measured on MI355X: 12288 x 3072
    weights 1.060 -> 0.846 ms with the 512 text rows as a second GEMM, 20-26 % less for each of
    the four shapes of a single block)."""
    return ((0, T), (T, N))


def _linear_rows(x, weight, bias, out, T, *, gelu=False):
    """out = x @ weight^T + bias (GELU(tanh) in the epilogue if ``gelu``), one GEMM per batch
    element and joint-sequence range, written in place into ``out``."""
    for b in range(x.shape[0]):
        for lo, hi in _joint_ranges(T, x.shape[1]):
            if gelu:
                torch._addmm_activation(bias, x[b, lo:hi], weight.t(), use_gelu=True, out=out[b, lo:hi])
            else:
                torch.addmm(bias, x[b, lo:hi], weight.t(), out=out[b, lo:hi])


class FluxTransformer:
    """Random-init FLUX.1-dev-shaped transformer; ``forward`` is one denoiser evaluation.

    Fused where the HIP path allows it, with the same arithmetic as the diffusers blocks up to
    rounding order: the text and image QKV projections of a double block write one joint
    [B, N, 3C] buffer (V is read from it in place), Q and K are normalised and rotated by one
    qk_prep_pair launch, every gated residual add is fused with the following AdaLN modulation
    (flux_norm.adaln_modulate; all blocks' modulation vectors depend only on the timestep
    embedding and are computed up front), the MLP GELU runs in the GEMM epilogue, and the single
    blocks' output projection over [attention | mlp] is two accumulating GEMMs instead of a
    concatenation.
    """

    def __init__(self, device, shape: FluxShape = FluxShape(), *, seed=0, dtype=torch.bfloat16):
        self.shape, self.device, self.dtype = shape, torch.device(device), dtype
        s, C, M = shape, shape.hidden, shape.mlp_hidden
        init = _Init(self.device, dtype, seed)
        self.x_embedder = init.linear(C, s.in_channels)
        self.context_embedder = init.linear(C, s.joint_attention_dim)
        self.time_embedder = init.mlp(s.timestep_dim, C)
        self.guidance_embedder = init.mlp(s.timestep_dim, C) if s.guidance_embeds else None
        self.text_embedder = init.mlp(s.pooled_projection_dim, C)
        # modulation weights are scaled down so the gated residual stream stays O(1) over 57 blocks
        mod_std = 0.2 * C**-0.5
        self.double = []
        for _ in range(s.num_layers):
            self.double.append(dict(
                mod_x=init.linear(6 * C, C, mod_std), mod_c=init.linear(6 * C, C, mod_std),
                qkv_x=init.linear(3 * C, C), qkv_c=init.linear(3 * C, C),
                norm_q=init.norm(s.head_dim), norm_k=init.norm(s.head_dim),
                norm_added_q=init.norm(s.head_dim), norm_added_k=init.norm(s.head_dim),
                out_x=init.linear(C, C), out_c=init.linear(C, C),
                ff_x=(init.linear(M, C), init.linear(C, M)), ff_c=(init.linear(M, C), init.linear(C, M)),
            ))
        self.single = []
        out_std = (C + M) ** -0.5
        for _ in range(s.num_single_layers):
            self.single.append(dict(
                mod=init.linear(3 * C, C, mod_std),
                qkv=init.linear(3 * C, C),                       # to_q | to_k | to_v
                mlp=init.linear(M, C),                           # proj_mlp
                norm_q=init.norm(s.head_dim), norm_k=init.norm(s.head_dim),
                out_attn=init.linear(C, C + M, out_std, out_features=C, in_features=C),
                out_mlp=init.linear(C, C + M, out_std, out_features=C, in_features=M, bias=False),
            ))
        self.norm_out = init.linear(2 * C, C, mod_std)
        self.proj_out = init.linear(s.in_channels, C)

    def parameters(self):
        def walk(x):
            if isinstance(x, torch.Tensor):
                yield x
            elif isinstance(x, (list, tuple)):
                for y in x:
                    yield from walk(y)
            elif isinstance(x, dict):
                for y in x.values():
                    yield from walk(y)

        for name in ("x_embedder", "context_embedder", "time_embedder", "guidance_embedder",
                     "text_embedder", "double", "single", "norm_out", "proj_out"):
            yield from walk(getattr(self, name))

    def parameter_count(self):
        return sum(p.numel() for p in self.parameters() if p is not None)

    # ------------------------------------------------------------------ blocks
    def _attend(self, attention, layer, q, k, v, out):
        """q/k/v/out are [B, N, H, D] storages; the kernels read them as [B, H, N, D] views."""
        attention(layer, q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), out.transpose(1, 2))

    def _modulations(self, silu_t):
        """Every block's AdaLN vectors (they depend on the timestep embedding only)."""
        double = [(F.linear(silu_t, *w["mod_x"]).chunk(6, dim=1), F.linear(silu_t, *w["mod_c"]).chunk(6, dim=1))
                  for w in self.double]
        single = [F.linear(silu_t, *w["mod"]).chunk(3, dim=1) for w in self.single]
        scale, shift = F.linear(silu_t, *self.norm_out).chunk(2, dim=1)   # AdaLayerNormContinuous order
        return double, single, (shift, scale)

    def _double_block(self, w, mods, x, xn, c, cn, cos, sin, attention, layer, next_mods, joint_out):
        """One double-stream block.  x / c are the residual streams, xn / cn their modulated rows
        (produced by the previous fused step).  Returns the updated (x, xn, c, cn); the residual
        add after the MLP is fused with the next block's modulation ``next_mods`` (shift, scale)
        pairs for image and text, or written into ``joint_out`` = (h, hn) [B, N, C] buffers when
        this is the last double block."""
        s, C, H = self.shape, self.shape.hidden, self.shape.heads
        B, n, _ = x.shape
        T = c.shape[1]
        (sx, scx, gx, sx2, scx2, gx2), (sc, scc, gc, sc2, scc2, gc2) = mods
        qkv = torch.empty(B, T + n, 3 * C, device=x.device, dtype=x.dtype)
        _linear_into(cn, *w["qkv_c"], qkv[:, :T])
        _linear_into(xn, *w["qkv_x"], qkv[:, T:])
        qk = qk_prep_pair(qkv[:, :T, :2 * C], qkv[:, T:, :2 * C], heads=H, eps=s.eps, cos=cos, sin=sin,
                          weights=((w["norm_added_q"], w["norm_q"]), (w["norm_added_k"], w["norm_k"])))
        v = qkv[..., 2 * C:].unflatten(-1, (H, s.head_dim))
        o = torch.empty_like(qk[0])
        self._attend(attention, layer, qk[0], qk[1], v, o)
        del qk, v, qkv
        o = o.view(B, T + n, C)
        ax = F.linear(o[:, T:], *w["out_x"])
        ac = F.linear(o[:, :T], *w["out_c"])
        del o
        xn = adaln_modulate(x, sx2, scx2, y=ax, gate=gx, x_out=x, eps=s.eps)
        cn = adaln_modulate(c, sc2, scc2, y=ac, gate=gc, x_out=c, eps=s.eps)
        del ax, ac
        (w1, b1), (w2, b2) = w["ff_x"]
        fx = F.linear(_gelu_linear(xn, w1, b1), w2, b2)
        (w1, b1), (w2, b2) = w["ff_c"]
        fc = F.linear(_gelu_linear(cn, w1, b1), w2, b2)
        if joint_out is None:
            (nsx, nscx), (nsc, nscc) = next_mods
            xn = adaln_modulate(x, nsx, nscx, y=fx, gate=gx2, x_out=x, eps=s.eps)
            cn = adaln_modulate(c, nsc, nscc, y=fc, gate=gc2, x_out=c, eps=s.eps)
            return x, xn, c, cn
        h, hn = joint_out
        nshift, nscale = next_mods
        adaln_modulate(x, nshift, nscale, y=fx, gate=gx2, x_out=h[:, T:], out=hn[:, T:], eps=s.eps)
        adaln_modulate(c, nshift, nscale, y=fc, gate=gc2, x_out=h[:, :T], out=hn[:, :T], eps=s.eps)
        return None

    def _single_block(self, w, mods, h, hn, T, cos, sin, attention, layer, next_mods):
        """One single-stream block over [text; image].  Returns (h, hn) with the residual add
        fused with the next block's modulation, or, for the last block, the image rows modulated
        by the output norm (``next_mods`` = norm_out's (shift, scale)) and no residual."""
        s, C, H = self.shape, self.shape.hidden, self.shape.heads
        B, N, _ = h.shape
        _, _, gate = mods
        qkv = hn.new_empty(B, N, 3 * C)                                    # to_q | to_k | to_v
        _linear_rows(hn, *w["qkv"], qkv, T)
        mlp = hn.new_empty(B, N, s.mlp_hidden)                            # GELU(proj_mlp)
        _linear_rows(hn, *w["mlp"], mlp, T, gelu=True)
        qk = qk_prep_pair(qkv[:, :T, :2 * C], qkv[:, T:, :2 * C], heads=H, eps=s.eps, cos=cos, sin=sin,
                          weights=((w["norm_q"], w["norm_q"]), (w["norm_k"], w["norm_k"])))
        v = qkv[..., 2 * C:].unflatten(-1, (H, s.head_dim))
        o = torch.empty_like(qk[0])
        self._attend(attention, layer, qk[0], qk[1], v, o)
        del qk, v, qkv
        (wa, ba), (wm, _) = w["out_attn"], w["out_mlp"]
        o = o.view(B, N, C)
        p = h.new_empty(B, N, C)                                           # proj_out([attn | mlp])
        for b in range(B):
            for lo, hi in _joint_ranges(T, N):
                pr = p[b, lo:hi]
                torch.addmm(ba, o[b, lo:hi], wa.t(), out=pr)
                pr.addmm_(mlp[b, lo:hi], wm.t())
        del o, mlp
        shift, scale = next_mods
        if layer < self.shape.blocks - 1:
            hn = adaln_modulate(h, shift, scale, y=p, gate=gate, x_out=h, eps=s.eps)
            return h, hn
        return None, adaln_modulate(h[:, T:], shift, scale, y=p[:, T:], gate=gate, eps=s.eps)

    # ------------------------------------------------------------------ forward
    def temb(self, timestep, guidance, pooled):
        s = self.shape
        t = timestep.to(self.dtype) * 1000
        emb = _mlp(timestep_projection(t, s.timestep_dim).to(self.dtype), self.time_embedder)
        if self.guidance_embedder is not None:
            g = guidance.to(self.dtype) * 1000
            emb = emb + _mlp(timestep_projection(g, s.timestep_dim).to(self.dtype), self.guidance_embedder)
        return emb + _mlp(pooled.to(self.dtype), self.text_embedder)

    @torch.inference_mode()
    def forward(self, hidden_states, encoder_hidden_states, pooled_projections, timestep, img_ids,
                txt_ids, guidance=None, *, attention=None, layout_scope="transformer"):
        """hidden_states [B, n, 64] packed latents, encoder_hidden_states [B, T, 4096],
        pooled_projections [B, 768], timestep [B], img_ids [n, 3], txt_ids [T, 3] -> predicted
        [B, n, 64].

        With a persistent layout, ``layout_scope="transformer"`` takes raster-order latents and
        ids and returns a raster-order prediction (one gather at entry and exit of this call,
        flux_adapter.py:209-212, :243); ``"sampling"`` takes latents and ids already in the plan's
        order and returns the prediction in that order (the permutation lives at the sampling
        loop's entry and exit instead, sampling_layout.py:88-116)."""
        s = self.shape
        if layout_scope not in ("transformer", "sampling"):
            raise ValueError("layout_scope must be transformer or sampling")
        attention = attention if attention is not None else NativeAttention()
        layout = attention.layout
        B, n, _ = hidden_states.shape
        T = encoder_hidden_states.shape[1]
        N = T + n
        if layout is not None:
            if N != layout.total_tokens:
                raise ValueError("token count does not match the plan")
            if layout_scope == "transformer":
                hidden_states = index_select_rows(hidden_states, 1, layout.order)
                img_ids = index_select_rows(img_ids.contiguous(), 0, layout.order)
        cos, sin = rotary_tables(torch.cat([txt_ids, img_ids]).to(self.device))
        double_mods, single_mods, out_mods = self._modulations(F.silu(self.temb(timestep, guidance,
                                                                                pooled_projections)))
        x = F.linear(hidden_states.to(self.dtype), *self.x_embedder)
        c = F.linear(encoder_hidden_states.to(self.dtype), *self.context_embedder)
        (sx, scx, *_), (sc, scc, *_) = double_mods[0]
        xn = adaln_modulate(x, sx, scx, eps=s.eps)
        cn = adaln_modulate(c, sc, scc, eps=s.eps)
        h = torch.empty(B, N, s.hidden, device=x.device, dtype=x.dtype)
        hn = torch.empty_like(h)
        for i, w in enumerate(self.double):
            last = i == len(self.double) - 1
            if last:
                nxt = single_mods[0][:2] if self.single else out_mods
                self._double_block(w, double_mods[i], x, xn, c, cn, cos, sin, attention, i, nxt, (h, hn))
            else:
                (nsx, nscx, *_), (nsc, nscc, *_) = double_mods[i + 1]
                x, xn, c, cn = self._double_block(w, double_mods[i], x, xn, c, cn, cos, sin, attention, i,
                                                  ((nsx, nscx), (nsc, nscc)), None)
        del x, xn, c, cn
        for j, w in enumerate(self.single):
            nxt = single_mods[j + 1][:2] if j + 1 < len(self.single) else out_mods
            h, hn = self._single_block(w, single_mods[j], h, hn, T, cos, sin, attention,
                                       s.num_layers + j, nxt)
        if hn.shape[1] != n:   # no single blocks: the last double block modulated every row
            hn = hn[:, T:]
        out = F.linear(hn, *self.proj_out)
        if layout is not None and layout_scope == "transformer":
            out = index_select_rows(out, 1, layout.inverse)
        return out

    __call__ = forward


def synthetic_inputs(device, *, grid, batch=1, text_tokens=512, shape: FluxShape = FluxShape(),
                     seed=0, timestep=0.5, guidance=3.5):
    """Seeded ~N(0,1) packed latents, text states and pooled embedding of FLUX's shapes, with the
    pipeline's position ids (text zeros, image (0, row, col) in raster order)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    n = grid * grid
    r, c = torch.meshgrid(torch.arange(grid), torch.arange(grid), indexing="ij")
    img_ids = torch.stack([torch.zeros(n), r.reshape(-1).float(), c.reshape(-1).float()], -1)
    args = dict(
        hidden_states=torch.randn(batch, n, shape.in_channels, generator=gen),
        encoder_hidden_states=torch.randn(batch, text_tokens, shape.joint_attention_dim, generator=gen),
        pooled_projections=torch.randn(batch, shape.pooled_projection_dim, generator=gen),
        timestep=torch.full((batch,), timestep),
        img_ids=img_ids,
        txt_ids=torch.zeros(text_tokens, 3),
        guidance=torch.full((batch,), guidance),
    )
    return {k: v.to(device=device, dtype=torch.bfloat16 if v.dtype == torch.float32 and v.ndim == 3 else v.dtype)
            for k, v in args.items()}
