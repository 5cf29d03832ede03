"""Drop-in BlockFHT API on MI355X.

Same public names, arguments and autograd behaviour as the reference module
``latent_weight_lab/block_fht.py``; every generated coordinate and every latent
gradient comes from the HIP library (``ops``).  Differences from the
reference, all widenings:

* float16 and bfloat16 latents run on the GPU (reference: float32 only,
  ``block_fht.py:161``).  Arithmetic is float32, except for bfloat16 latents of
  block 2^15, which run on the matrix cores: bf16 operands at every radix-32
  stage (9 roundings at 3 layers), float32 accumulation;
* blocks of any size 2^0 .. 2^23 (reference CUDA: 2^5 .. 2^23);
* the fused linear keeps the reference's own domain (float32 / float16 /
  bfloat16, ``block_size <= 2^14``, ``block_size % in_features == 0``,
  ``block_fht.py:263-273``) and adds bf16 latents of block 2^15 with
  ``in_features % 8 == 0`` in 528..5120, rows straddling blocks (matrix cores);
  several matrices can run in one grouped call (``forward_fused_grouped``);
* latent gradients are summed over blocks in a fixed order (deterministic).

There is no CPU path: CPU tensors raise RuntimeError.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from . import _native
from . import ops

next_power_of_two = ops.next_power_of_two

_MASK32 = 0xFFFFFFFF


def lowbias32(x: int) -> int:
    """32-bit avalanche hash (reference ``block_fht.py:36-43``)."""
    x &= _MASK32
    for shift, mult in ((16, 0x7FEB352D), (15, 0x846CA68B)):
        x = ((x ^ (x >> shift)) * mult) & _MASK32
    return x ^ (x >> 16)


def sign_word_for(seed: int, block: int, layer: int, word: int) -> int:
    """Sign bits of positions ``32*word .. 32*word+31`` of (block, layer)
    (reference ``block_fht.py:46-52``).  Bit set = +1."""
    seed = int(seed)
    mixed = (seed ^ (seed >> 32)) & _MASK32
    for const, value in ((0x9E3779B9, block), (0x85EBCA6B, layer), (0xC2B2AE35, word)):
        mixed ^= (const * (int(value) + 1)) & _MASK32
    return lowbias32(mixed)


def signs_for(reference: torch.Tensor, block: int, layer: int, seed: int, block_size: int) -> torch.Tensor:
    """+-1 vector of length ``block_size`` in ``reference``'s dtype and device
    (reference ``block_fht.py:55-81``), from the device hash."""
    _native.require_cuda(reference)
    words = ops.sign_words(seed, block, layer, (int(block_size) + 31) // 32, device=reference.device)
    bits = (words.to(torch.int64).unsqueeze(1) >> torch.arange(32, device=reference.device)) & 1
    return (2.0 * bits.reshape(-1)[: int(block_size)] - 1.0).to(dtype=reference.dtype)


class _BlockFHTSliceFn(torch.autograd.Function):
    """Reference ``block_fht.py:149-196`` with the HIP library in both directions."""

    @staticmethod
    def forward(ctx, latent, size, layers, seed, start, stop):
        latent = latent.contiguous()
        ctx.latent_size = latent.numel()
        ctx.latent_dtype = latent.dtype
        ctx.args = (int(size), int(layers), int(seed), int(start), int(stop))
        return ops.forward(latent, *ctx.args)

    @staticmethod
    def backward(ctx, grad_out):
        size, layers, seed, start, stop = ctx.args
        grad = ops.backward(grad_out, ctx.latent_size, ctx.latent_dtype, size, layers, seed, start, stop)
        return grad, None, None, None, None, None


def block_fht_slice(latent: torch.Tensor, size: int, layers: int, seed: int, start: int, stop: int) -> torch.Tensor:
    """Generated coordinates ``[start, stop)`` (reference ``block_fht.py:199-207``)."""
    return _BlockFHTSliceFn.apply(latent, int(size), int(layers), int(seed), int(start), int(stop))


def block_fht_grad_latent(latent: torch.Tensor, grad_out: torch.Tensor, size: int, layers: int, seed: int,
                          start: int = 0, stop: int | None = None) -> torch.Tensor:
    """Latent gradient of ``block_fht_slice`` for a given output gradient
    (reference ``block_fht.py:210-248``)."""
    stop = int(size) if stop is None else int(stop)
    _native.require_cuda(latent, grad_out)
    return ops.backward(grad_out, latent.numel(), latent.dtype, int(size), int(layers), int(seed), int(start), stop)


def block_fht_linear_forward(input: torch.Tensor, latent: torch.Tensor, out_features: int, layers: int, seed: int,
                             weight_scale: float = 1.0, fused: bool | None = None) -> torch.Tensor:
    """``input @ (weight_scale * W)^T`` with ``W = BlockFHT(latent)[: in*out].view(out, in)``
    (reference ``block_fht.py:251-288``).

    Two routes.  The fused one, for shapes a fused kernel takes — the reference's own
    domain (float32 / float16 / bfloat16 latents of block <= 2^14 with ``block %
    in_features == 0``), and bf16 latents of block 2^15 with ``in_features % 8 == 0`` in
    528..5120 — generates W on chip for every token range and contracts it there, so only
    the latent and the activations live in HBM.  The other generates W once into a
    transient buffer (one launch, ``weight_scale`` folded in) and calls ``F.linear`` — the
    reference's fallback (``:282-288``), which the reference also takes at every block-2^15
    shape.  ``fused=True`` takes the fused route wherever a kernel takes the shape,
    ``fused=False`` never; the default (None) takes it where it is also the faster one:
    small batches (``ops.linear_fused_preferred``: below 128 tokens on the block-2^15
    kernel, below 8 in the reference's domain).  At decode batch sizes
    ``forward_fused_grouped`` runs many matrices' fused kernels together.  Both routes are
    differentiable in the input and the latent, as the reference's fallback is: the fused
    one through ``_FusedLinearFn`` (W regenerated in the backward), the other through
    ``block_fht_slice``.
    """
    return _generated_linear(input, latent, out_features, layers, seed, weight_scale, None, fused)


def _generated_linear(input, latent, out_features, layers, seed, weight_scale, bias, fused):
    # block_fht_linear_forward, with an optional bias added by the GEMM's epilogue
    if input.dim() < 2:
        raise ValueError("input must have at least 2 dimensions")
    in_features = int(input.shape[-1])
    out_features = int(out_features)
    flat = input.reshape(-1, in_features)
    _native.require_cuda(flat, latent)
    size = in_features * out_features
    use_fused = (ops.linear_fused_preferred(in_features, out_features, latent, flat) if fused is None
                 else bool(fused) and ops.linear_supported(in_features, out_features, latent, flat))
    if use_fused:
        if torch.is_grad_enabled() and (latent.requires_grad or flat.requires_grad):
            out = _FusedLinearFn.apply(flat, latent, out_features, int(layers), int(seed), float(weight_scale))
        else:
            out = ops.linear_forward(flat, latent, out_features, int(layers), int(seed), float(weight_scale))
        if bias is not None:
            out = out + bias
    elif torch.is_grad_enabled() and latent.requires_grad:
        weight = block_fht_slice(latent, size, int(layers), int(seed), 0, size).view(out_features, in_features)
        out = F.linear(flat.contiguous(), weight * float(weight_scale), bias)
    else:
        with torch.no_grad():
            if ops.weight_job_supported(latent, size, int(layers), latent.dtype):
                (weight,) = ops.materialize_weights([(latent, size, int(layers), int(seed), float(weight_scale),
                                                      latent.dtype)])
            else:
                weight = block_fht_slice(latent, size, int(layers), int(seed), 0, size) * float(weight_scale)
        out = F.linear(flat.contiguous(), weight.view(out_features, in_features), bias)
    return out.reshape(*input.shape[:-1], out_features)


class _FusedLinearFn(torch.autograd.Function):
    """The fused route of ``block_fht_linear_forward`` with the gradients of the
    reference's differentiable fallback (``block_fht.py:282-288``: W from
    ``block_fht_slice``, ``* weight_scale``, ``F.linear``).  The forward keeps W on
    chip; the backward regenerates ``weight_scale * W`` once (one grouped launch)
    for ``grad_input = g W`` and projects ``grad_weight = g^T x`` onto the latent
    through the generator's backward, as ``_BlockFHTLinearFn.backward`` does
    (reference ``:330-350``)."""

    @staticmethod
    def forward(ctx, x2d, latent, out_features, layers, seed, weight_scale):
        ctx.save_for_backward(x2d, latent)
        ctx.meta = (int(out_features), int(layers), int(seed), float(weight_scale))
        return ops.linear_forward(x2d, latent, out_features, layers, seed, weight_scale)

    @staticmethod
    def backward(ctx, grad_out):
        x2d, latent = ctx.saved_tensors
        out_f, layers, seed, scale = ctx.meta
        in_f = int(x2d.shape[1])
        size = in_f * out_f
        g = grad_out.reshape(-1, out_f)
        grad_x = grad_latent = None
        if ctx.needs_input_grad[0]:
            with torch.no_grad():
                lat = latent.detach()
                if ops.weight_job_supported(lat, size, layers, lat.dtype):
                    (w,) = ops.materialize_weights([(lat, size, layers, seed, scale, lat.dtype)])
                else:
                    w = block_fht_slice(lat, size, layers, seed, 0, size) * scale
            grad_x = g.to(dtype=w.dtype).matmul(w.view(out_f, in_f)).to(dtype=x2d.dtype)
        if ctx.needs_input_grad[1]:
            grad_weight = g.t().to(dtype=latent.dtype).matmul(x2d.to(dtype=latent.dtype))
            grad_latent = scale * block_fht_grad_latent(latent.detach(), grad_weight.reshape(-1), size, layers, seed)
        return grad_x, grad_latent, None, None, None, None


class _BlockFHTLinearFn(torch.autograd.Function):
    """Training linear (reference ``block_fht.py:291-356``): W is generated for
    the forward and again for grad_input; grad_latent goes through the HIP
    backward of the generator, with grad_weight = g^T x either on a library GEMM
    (the reference's route, and its rounding) or, with ``fused_latent_grad``, in
    one call of the library's latent-gradient entry (its own split-K matrix-core
    GEMM into float32 partials, then the generator's backward: faster at config-4
    shapes; grad_weight is rounded once, after weight_scale)."""

    @staticmethod
    def forward(ctx, input, latent, bias, in_features, out_features, size, layers, seed, weight_scale,
                modulation_alpha, fused_latent_grad=False):
        weight = _generated_weight(latent, size, layers, seed, weight_scale, modulation_alpha)
        weight = weight.view(int(out_features), int(in_features)).to(dtype=input.dtype)
        ctx.save_for_backward(input, latent)
        ctx.has_bias = bias is not None
        ctx.meta = (int(in_features), int(out_features), int(size), int(layers), int(seed), float(weight_scale),
                    float(modulation_alpha))
        ctx.fused_latent_grad = bool(fused_latent_grad)
        return F.linear(input, weight, bias)

    @staticmethod
    def backward(ctx, grad_output):
        input, latent = ctx.saved_tensors
        in_f, out_f, size, layers, seed, scale, alpha = ctx.meta
        grad_2d = grad_output.reshape(-1, out_f)
        grad_input = grad_latent = grad_bias = None
        if ctx.needs_input_grad[0]:
            with torch.no_grad():
                weight = _generated_weight(latent, size, layers, seed, scale, alpha)
                weight = weight.view(out_f, in_f).to(dtype=grad_output.dtype)
            grad_input = grad_2d.matmul(weight).reshape_as(input)
        if ctx.needs_input_grad[1]:
            input_2d = input.reshape(-1, in_f)
            g = grad_2d.to(dtype=latent.dtype)
            xl = input_2d.to(dtype=latent.dtype)
            if (ctx.fused_latent_grad and size == in_f * out_f
                    and ops.linear_backward_latent_supported(in_f, out_f, latent, xl, g)):
                # grad_weight = g^T x and the generator's backward in one library call
                grad_latent = ops.linear_backward_latent(g, xl, latent, out_f, layers, seed, scale)
                if alpha != 0.0:  # sum of grad_weight = sum_t (sum_o g[t, o]) (sum_i x[t, i])
                    gw_sum = (g.float().sum(dim=1) * xl.float().sum(dim=1)).sum()
                    grad_latent = grad_latent + (2.0 * alpha * gw_sum * latent.float()).to(latent.dtype)
            else:
                grad_weight = g.t().matmul(xl)
                grad_latent = scale * block_fht_grad_latent(latent, grad_weight.reshape(-1), size, layers, seed)
                if alpha != 0.0:
                    grad_latent = grad_latent + 2.0 * alpha * latent * grad_weight.sum()
        if ctx.has_bias and ctx.needs_input_grad[2]:
            grad_bias = grad_2d.sum(dim=0).to(dtype=grad_output.dtype)
        return grad_input, grad_latent, grad_bias, None, None, None, None, None, None, None, None


def _generated_weight(latent, size, layers, seed, weight_scale, modulation_alpha):
    flat = block_fht_slice(latent, int(size), int(layers), int(seed), 0, int(size)) * float(weight_scale)
    if float(modulation_alpha) != 0.0:
        flat = flat + float(modulation_alpha) * latent.square().sum()
    return flat


def _walsh_columns(length: int, rank: int, seed: int) -> torch.Tensor:
    """Columns ``seed .. seed+rank-1`` of the Sylvester Hadamard matrix of
    order ``length`` (rows truncated), scaled by 1/sqrt(length)
    (reference ``block_fht.py:426-435``)."""
    rows = torch.arange(length, dtype=torch.int64).view(-1, 1)
    cols = (torch.arange(rank, dtype=torch.int64) + int(seed)).view(1, -1)
    bits = rows & cols
    parity = torch.zeros_like(bits)
    while bool(bits.any()):
        parity ^= bits & 1
        bits = bits >> 1
    return (1.0 - 2.0 * parity.float()) / math.sqrt(length)


class BlockFHTLinear(nn.Module):
    """Linear layer whose weight is generated by BlockFHT (reference
    ``block_fht.py:359-557``), with the same options: bias, latent_dim /
    latent_ratio, weight_scale, norm modulation, residual base, per-channel
    gains, spectral correction, and the materialized weight cache."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False, latent_dim: int | None = None,
                 latent_ratio: float = 0.01, layers: int = 3, seed: int = 0, latent_init_std: float = 0.02,
                 weight_scale: float = 1.0, modulation_alpha: float = 0.0, modulation_centered: bool = False,
                 residual_base_scale: float = 0.0, residual_base_std: float = 0.02, output_gain: bool = False,
                 input_gain: bool = False, spectral_rank: int = 0, spectral_out_groups: int = 1,
                 spectral_in_groups: int = 1, fused_latent_grad: bool = False) -> None:
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        size = self.in_features * self.out_features
        if latent_dim is None:
            latent_dim = max(1, round(size * float(latent_ratio)))
        self.generator = BlockFHT(int(latent_dim), size=size, layers=layers, seed=seed,
                                  latent_init_std=latent_init_std)
        self.bias = nn.Parameter(torch.zeros(self.out_features)) if bias else None
        self._cached_weight: torch.Tensor | None = None
        self.weight_scale = float(weight_scale)
        self.modulation_alpha = float(modulation_alpha)
        self.modulation_centered = bool(modulation_centered)
        # not in the reference: the latent gradient in one library call
        # (lwl_bfht_linear_backward_latent) instead of a library GEMM + the backward
        self.fused_latent_grad = bool(fused_latent_grad)
        self.latent_init_std = float(latent_init_std)
        self.residual_base_scale = float(residual_base_scale)
        self.output_gain = nn.Parameter(torch.ones(self.out_features)) if output_gain else None
        self.input_gain = nn.Parameter(torch.ones(self.in_features)) if input_gain else None
        self.spectral_rank = int(spectral_rank)
        self.spectral_out_groups = int(spectral_out_groups)
        self.spectral_in_groups = int(spectral_in_groups)
        if self.spectral_rank:
            if self.spectral_rank > min(self.in_features, self.out_features):
                raise ValueError("spectral_rank exceeds matrix dimensions")
            if self.out_features % self.spectral_out_groups or self.in_features % self.spectral_in_groups:
                raise ValueError("spectral gain groups must divide feature dimensions")
            self.register_buffer("spectral_u", _walsh_columns(self.out_features, self.spectral_rank, seed + 17),
                                 persistent=True)
            self.register_buffer("spectral_v", _walsh_columns(self.in_features, self.spectral_rank, seed + 31),
                                 persistent=True)
            self.spectral_core = nn.Parameter(torch.zeros(self.spectral_rank, self.spectral_rank))
            self.spectral_log_out_gain = nn.Parameter(torch.zeros(self.spectral_out_groups))
            self.spectral_log_in_gain = nn.Parameter(torch.zeros(self.spectral_in_groups))
        else:
            self.spectral_u = self.spectral_v = None
            self.spectral_core = self.spectral_log_out_gain = self.spectral_log_in_gain = None
        if self.residual_base_scale != 0.0:
            base = torch.empty(self.out_features, self.in_features)
            nn.init.normal_(base, mean=0.0, std=float(residual_base_std))
            self.register_buffer("residual_base_weight", base, persistent=True)
        else:
            self.residual_base_weight = None

    _hadamard_columns = staticmethod(_walsh_columns)

    def _modulation_offset(self) -> torch.Tensor:
        offset = self.generator.latent.square().sum()
        if self.modulation_centered:
            expected = self.generator.latent.numel() * self.latent_init_std * self.latent_init_std
            offset = offset - offset.new_tensor(expected)
        return offset

    def _needs_dense_path(self) -> bool:
        return (self.residual_base_weight is not None or self.modulation_centered or self.output_gain is not None
                or self.input_gain is not None or self.spectral_core is not None)

    @property
    def weight(self) -> torch.Tensor:
        """The generated weight with every option applied (reference ``block_fht.py:444-462``)."""
        return self._finish_weight(self.generator() * self.weight_scale)

    def _finish_weight(self, weight: torch.Tensor) -> torch.Tensor:
        """Every option after ``generator() * weight_scale`` (flat, latent dtype)."""
        if self.modulation_alpha != 0.0:
            weight = weight + self.modulation_alpha * self._modulation_offset()
        weight = weight.view(self.out_features, self.in_features)
        if self.residual_base_weight is not None:
            base = self.residual_base_weight.to(device=weight.device, dtype=weight.dtype)
            weight = base + self.residual_base_scale * weight
        if self.spectral_core is not None:
            dt = weight.dtype
            correction = self.spectral_u.to(dtype=dt) @ self.spectral_core.to(dtype=dt) @ self.spectral_v.to(dtype=dt).t()
            weight = weight + correction
            out_gain = self.spectral_log_out_gain.exp().repeat_interleave(self.out_features // self.spectral_out_groups)
            in_gain = self.spectral_log_in_gain.exp().repeat_interleave(self.in_features // self.spectral_in_groups)
            weight = weight * out_gain.to(dtype=dt).view(-1, 1) * in_gain.to(dtype=dt).view(1, -1)
        if self.output_gain is not None:
            weight = weight * self.output_gain.to(device=weight.device, dtype=weight.dtype).view(-1, 1)
        if self.input_gain is not None:
            weight = weight * self.input_gain.to(device=weight.device, dtype=weight.dtype).view(1, -1)
        return weight

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if self._cached_weight is not None:
            return F.linear(input, self._cached_weight, self.bias)
        if self._needs_dense_path():
            return F.linear(input, self.weight.to(dtype=input.dtype), self.bias)
        g = self.generator
        return _BlockFHTLinearFn.apply(input, g.latent, self.bias, self.in_features, self.out_features, g.size,
                                       g.layers, g.seed, self.weight_scale, self.modulation_alpha,
                                       self.fused_latent_grad)

    def forward_fused(self, input: torch.Tensor, weight_scale: float = 1.0) -> torch.Tensor:
        """Inference forward (reference ``block_fht.py:482-501``).  Where the default route
        of ``block_fht_linear_forward`` is the fused kernel (it takes the shape and the
        batch is small, ``ops.linear_fused_preferred``) and no gradient is recorded: one
        fused launch whose stores also add the modulation term, the residual base and the
        bias (``lwl_bfht_linear_forward_ex``; W never stored, one rounding to the output
        dtype instead of one per term).  Otherwise: that route's linear (fused or W
        generated once) with the reference's sequence of terms after it, the bias in the
        GEMM's epilogue when nothing comes between."""
        if self.output_gain is not None or self.input_gain is not None or self.spectral_core is not None:
            return F.linear(input, self.weight.to(dtype=input.dtype), self.bias)
        g = self.generator
        scale = weight_scale * self.weight_scale
        fused = self._fused_epilogue_args(input, scale)
        if fused is not None:
            flat, args, kwargs = fused
            return ops.linear_forward(flat, *args, **kwargs).reshape(*input.shape[:-1], self.out_features)
        if self.modulation_alpha == 0.0 and self.residual_base_weight is None:
            # the bias rides in the GEMM's epilogue
            return _generated_linear(input, g.latent, self.out_features, g.layers, g.seed, scale, self.bias, None)
        out = block_fht_linear_forward(input, g.latent, self.out_features, g.layers, g.seed, weight_scale=scale)
        if self.modulation_alpha != 0.0:
            modulation = self.modulation_alpha * self._modulation_offset()
            out = out + modulation.to(dtype=out.dtype) * input.sum(dim=-1, keepdim=True)
        if self.residual_base_weight is not None:
            base_out = F.linear(input, self.residual_base_weight.to(device=input.device, dtype=input.dtype))
            out = base_out + self.residual_base_scale * out
        if self.bias is not None:
            out = out + self.bias
        return out

    def _fused_epilogue_args(self, input: torch.Tensor, scale: float):
        """``(flat input, ops.linear_forward positional args, epilogue kwargs)`` of
        ``forward_fused`` as one fused launch, or None where that route does not apply
        (gradients recorded, no fused kernel for the shape, a bias of another dtype).
        The terms follow the reference's tail (``block_fht.py:493-500``): with a residual
        base, ``out = base + s * (x W'^T + m * x.sum(-1))`` (s = residual_base_scale,
        folded into weight_scale and the row-sum factor), then ``+ bias``; m is the
        modulation rounded to the output dtype, as the reference rounds it."""
        g = self.generator
        if input.dim() < 2 or not (input.is_cuda and g.latent.is_cuda):
            return None
        bias = self.bias
        if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (g.latent, input, bias)):
            return None
        flat = input.reshape(-1, self.in_features)
        if not ops.linear_fused_preferred(self.in_features, self.out_features, g.latent, flat):
            return None
        if bias is not None and bias.dtype != flat.dtype:
            return None
        kwargs = {}
        if bias is not None:
            kwargs["bias"] = bias.detach()
        out_scale = 1.0
        if self.residual_base_weight is not None:
            base_weight = self.residual_base_weight.to(device=flat.device, dtype=flat.dtype)
            kwargs["base"] = F.linear(flat, base_weight)
            out_scale = self.residual_base_scale
        if self.modulation_alpha != 0.0:
            kwargs["row_sum_coef"] = (self.modulation_alpha * self._modulation_offset()).detach().to(dtype=flat.dtype)
            kwargs["row_sum_scale"] = out_scale
        args = (g.latent, self.out_features, g.layers, g.seed, scale * out_scale)
        return flat, args, kwargs

    def materialize_weight_cache(self, dtype: torch.dtype | None = None) -> None:
        """Reference ``block_fht.py:503-512``."""
        if self.residual_base_weight is not None or self.spectral_core is not None or self._cached_weight is not None:
            return
        with torch.no_grad():
            weight = self.weight
            if dtype is not None:
                weight = weight.to(dtype=dtype)
        self._cached_weight = weight.detach().requires_grad_(True)

    def flush_weight_cache_to_latent_grad(self) -> None:
        """Project the cached weight's gradient back onto the latent (and the
        gains) and drop the cache (reference ``block_fht.py:514-557``)."""
        if self._cached_weight is None:
            return
        if self._cached_weight.grad is not None:
            g = self.generator
            generated_grad = self._generated_weight_grad()
            grad_latent = self.weight_scale * block_fht_grad_latent(g.latent, generated_grad, g.size, g.layers, g.seed)
            self._add_latent_grad(grad_latent, generated_grad)
        self._cached_weight = None

    def _generated_weight_grad(self) -> torch.Tensor:
        """Gradient of the cached weight with respect to the generated one (flat,
        latent dtype); accumulates the gains' gradients on the way."""
        latent = self.generator.latent
        grad_weight = self._cached_weight.grad.to(dtype=latent.dtype)
        cached = self._cached_weight.detach().to(dtype=latent.dtype)
        generated_grad = grad_weight
        for gain, dim, view in ((self.output_gain, 1, (-1, 1)), (self.input_gain, 0, (1, -1))):
            if gain is None:
                continue
            gd = gain.detach().to(dtype=latent.dtype)
            if torch.any(gd == 0):
                which = "output" if dim == 1 else "input"
                raise RuntimeError(f"cannot flush a cached BlockFHT weight with a zero {which} gain")
            gain_grad = (grad_weight * (cached / gd.view(*view))).sum(dim=dim).to(dtype=gain.dtype)
            if gain.grad is None:
                gain.grad = gain_grad
            else:
                gain.grad.add_(gain_grad)
            generated_grad = generated_grad * gd.view(*view)
        generated_grad = generated_grad.reshape(-1)
        if self.residual_base_weight is not None:
            generated_grad = generated_grad * self.residual_base_scale
        return generated_grad

    def _add_latent_grad(self, grad_latent: torch.Tensor, generated_grad: torch.Tensor) -> None:
        latent = self.generator.latent
        if self.modulation_alpha != 0.0:
            grad_latent = grad_latent + 2.0 * self.modulation_alpha * latent * generated_grad.sum()
        if latent.grad is None:
            latent.grad = grad_latent
        else:
            latent.grad.add_(grad_latent)

    def _cache_needs_torch_epilogue(self) -> bool:
        # options applied in torch around the grouped kernels (the plain case
        # scales, casts and accumulates inside them)
        return self.modulation_alpha != 0.0 or self.output_gain is not None or self.input_gain is not None


def forward_fused_grouped(modules: list["BlockFHTLinear"], inputs: list[torch.Tensor],
                          weight_scale: float = 1.0) -> list[torch.Tensor]:
    """``[m.forward_fused(x, weight_scale) for m, x in zip(modules, inputs)]`` in one
    grouped fused-linear call (``lwl_bfht_linear_forward_grouped``) for every module that
    ``forward_fused`` would run as one fused launch: at decode batch sizes one matrix fills
    a fraction of the chip, and the grouped launch runs all of them together (not in the
    reference, which calls ``ext.linear_forward`` per matrix, ``block_fht.py:274``).  Each
    job carries its module's epilogue (bias in the grouped kernels; modulation or residual
    base make it a single launch inside the call).  Outputs equal the per-module calls bit
    for bit.  Other modules, and calls that record gradients, run ``forward_fused`` one
    by one."""
    if len(modules) != len(inputs):
        raise ValueError("modules and inputs must have the same length")
    outs: list[torch.Tensor | None] = [None] * len(modules)
    grouped, specs = [], []
    for i, (m, x) in enumerate(zip(modules, inputs)):
        direct = not (m.output_gain is not None or m.input_gain is not None or m.spectral_core is not None)
        fused = m._fused_epilogue_args(x, weight_scale * m.weight_scale) if direct else None
        if fused is not None and (not specs or fused[0].dtype == specs[0][0].dtype):
            flat, args, kwargs = fused
            grouped.append(i)
            specs.append((flat, *args, kwargs))
        else:
            outs[i] = m.forward_fused(x, weight_scale=weight_scale)
    if specs:
        for i, y in zip(grouped, ops.linear_forward_grouped(specs)):
            outs[i] = y.reshape(*inputs[i].shape[:-1], modules[i].out_features)
    return outs


def _cacheable(module: "BlockFHTLinear") -> bool:
    return (module.residual_base_weight is None and module.spectral_core is None
            and module._cached_weight is None)


def prepare_block_fht_weight_cache(model: nn.Module, dtype: torch.dtype | None = None) -> None:
    """Materialize every BlockFHTLinear's weight once (reference ``block_fht.py:560-563``).

    The generators run together in a few grouped launches (``ops.materialize_weights``);
    a module the grouped kernels do not take (blocks above 2^15, a bfloat16 latent of
    block 2^15 cached in another dtype) materializes on its own.  The cached weights
    are bit-identical either way.
    """
    grouped, specs = [], []
    for module in model.modules():
        if not isinstance(module, BlockFHTLinear) or not _cacheable(module):
            continue
        g = module.generator
        latent = g.latent
        plain = not module._cache_needs_torch_epilogue()
        # the kernel's output dtype: the cache dtype when it finishes the weight
        wdtype = (dtype or latent.dtype) if plain else latent.dtype
        if ops.weight_job_supported(latent, g.size, g.layers, wdtype):
            grouped.append((module, plain))
            specs.append((latent, g.size, g.layers, g.seed, module.weight_scale, wdtype))
        else:
            module.materialize_weight_cache(dtype=dtype)
    if not specs:
        return
    with torch.no_grad():
        weights = ops.materialize_weights(specs)
        for (module, plain), w in zip(grouped, weights):
            if not plain:
                w = module._finish_weight(w)
                if dtype is not None:
                    w = w.to(dtype=dtype)
            module._cached_weight = w.view(module.out_features, module.in_features).detach().requires_grad_(True)


def flush_block_fht_weight_cache(model: nn.Module) -> None:
    """Project every cached weight's gradient onto its latent and drop the caches
    (reference ``block_fht.py:566-569``).

    All generators' adjoints run in a few grouped launches (``ops.flush_weight_grads``),
    which also scale by weight_scale and add into ``latent.grad``; gains and
    modulation are applied in torch around them, as in the per-module flush.
    """
    grouped, specs, targets = [], [], set()
    for module in model.modules():
        if not isinstance(module, BlockFHTLinear) or module._cached_weight is None:
            continue
        cached = module._cached_weight
        if cached.grad is None:
            module._cached_weight = None
            continue
        g = module.generator
        latent = g.latent
        plain = not module._cache_needs_torch_epilogue()
        if plain:
            source = cached.grad.contiguous().reshape(-1)
            supported = ops.weight_job_supported(latent, g.size, g.layers, source.dtype, source)
        else:
            # the source is the generated-weight gradient in the latent dtype
            supported = ops.weight_job_supported(latent, g.size, g.layers, latent.dtype)
        if not supported:
            module.flush_weight_cache_to_latent_grad()
            continue
        if not plain:
            source = module._generated_weight_grad()
        into = None
        if (plain and latent.grad is not None and latent.grad.is_contiguous() and latent.grad.dtype == latent.dtype
                and id(latent) not in targets):
            into = latent.grad  # the kernel adds in place (a latent shared by modules: the first only)
        targets.add(id(latent))
        grouped.append((module, plain, source, into))
        specs.append((latent, source, g.size, g.layers, g.seed, module.weight_scale, into))
    if not specs:
        return
    with torch.no_grad():
        results = ops.flush_weight_grads(specs)
    for (module, plain, source, into), r in zip(grouped, results):
        latent = module.generator.latent
        if into is not None:
            pass  # added in place
        elif plain:
            if latent.grad is None:
                latent.grad = r
            else:
                latent.grad.add_(r)
        else:
            module._add_latent_grad(r, source)
        module._cached_weight = None


def suspend_block_fht_weight_cache(model: nn.Module) -> list[tuple[BlockFHTLinear, torch.Tensor]]:
    """Detach live caches so a forward sees the live latent; the handles keep
    the cached leaves and their gradients (reference ``block_fht.py:572-586``)."""
    suspended = []
    for module in model.modules():
        if isinstance(module, BlockFHTLinear) and module._cached_weight is not None:
            suspended.append((module, module._cached_weight))
            module._cached_weight = None
    return suspended


def restore_block_fht_weight_cache(suspended: list[tuple[BlockFHTLinear, torch.Tensor]]) -> None:
    """Reference ``block_fht.py:589-594``."""
    for module, weight in suspended:
        if module._cached_weight is not None:
            raise RuntimeError("cannot restore BlockFHT cache over a live cached weight")
        module._cached_weight = weight


class BlockFHT(nn.Module):
    """Latent -> generated vector of length ``size`` (reference ``block_fht.py:597-641``)."""

    def __init__(self, latent: int | torch.Tensor | nn.Parameter, size: int, layers: int = 3, seed: int = 0,
                 latent_init_std: float = 0.02) -> None:
        super().__init__()
        if size <= 0:
            raise ValueError("size must be positive")
        if layers not in {1, 2, 3}:
            raise ValueError("layers must be 1, 2, or 3")
        if isinstance(latent, int):
            if latent <= 0:
                raise ValueError("latent size must be positive")
            self.latent_size = int(latent)
            self.latent = nn.Parameter(torch.empty(self.latent_size))
            nn.init.normal_(self.latent, std=float(latent_init_std))
        else:
            if latent.dim() != 1:
                raise ValueError("latent tensor must be 1D")
            self.latent_size = int(latent.numel())
            self.latent = latent if isinstance(latent, nn.Parameter) else nn.Parameter(latent)
        self.size = int(size)
        self.layers = int(layers)
        self.seed = int(seed)
        self.block_size = next_power_of_two(self.latent_size)

    def extra_repr(self) -> str:
        return (f"latent_size={self.latent_size}, size={self.size}, layers={self.layers}, "
                f"seed={self.seed}, block_size={self.block_size}")

    def slice(self, start: int, stop: int) -> torch.Tensor:
        return block_fht_slice(self.latent, self.size, self.layers, self.seed, start, stop)

    def forward(self) -> torch.Tensor:
        return self.slice(0, self.size)

    @property
    def cuda_extension_error(self) -> Exception | None:
        """Why the HIP library could not load (None when it is loaded)."""
        return _native.load_error()
