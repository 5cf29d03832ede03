"""Many small generators in one launch: linears built from several BlockFHTLinear
heads (the nanoGPT example's ``HeadwiseLinear`` and ``GroupedInputLinear``,
reference ``examples/nanogpt/model.py:136-175,241-277``), whose heads each call
the generator separately in the reference (one ``ext.forward`` per head in the
forward, one more for grad_input and one ``ext.backward`` per head).

Here every head's weight comes out of one grouped generation
(``ops.materialize_weights``) straight into the concatenated matrix, and every
head's latent gradient out of one grouped adjoint (``ops.flush_weight_grads``).
Per head the arithmetic is that of ``BlockFHTLinear.forward``
(``_BlockFHTLinearFn``): the weight ``T(T(gen) * weight_scale)`` cast to the
input dtype, grad_weight = gᵀx in the latent dtype, grad_latent = weight_scale ·
Tᵀ(grad_weight).  Heads outside that plain form (gains, residual base,
spectral correction, norm modulation, a live weight cache, or latents the
grouped kernels do not take) run head by head, exactly as the reference does.
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as F

from . import _native
from . import ops
from .block_fht import BlockFHTLinear


def _plain(head: BlockFHTLinear) -> bool:
    return (isinstance(head, BlockFHTLinear) and head._cached_weight is None and not head._needs_dense_path()
            and head.modulation_alpha == 0.0)


def _batchable(heads: Sequence[BlockFHTLinear], dtype: torch.dtype) -> bool:
    if not heads or not all(_plain(h) for h in heads):
        return False
    lat0 = heads[0].generator.latent
    if not lat0.is_cuda:
        return False
    for h in heads:
        g = h.generator
        if g.latent.dtype != lat0.dtype or g.latent.device != lat0.device or g.size != h.in_features * h.out_features:
            return False
        if not ops.weight_job_supported(g.latent, g.size, g.layers, dtype):
            return False
    return True


def _weight(heads, latents, dtype, layout):
    """The concatenated weight, every head generated in one grouped launch (latent dtype
    rounding, scale, cast).  Row layout ([sum out, in]): the heads' weights are
    consecutive row blocks, generated in place; column layout ([out, sum in]): generated
    head by head into a staging buffer, then interleaved."""
    kernel_dtype = dtype
    if not all(ops.weight_job_supported(lat, h.generator.size, h.generator.layers, dtype)
               for h, lat in zip(heads, latents)):
        kernel_dtype = latents[0].dtype  # always taken; the cast follows in torch
    specs = [(lat, h.generator.size, h.generator.layers, h.generator.seed, h.weight_scale, kernel_dtype)
             for h, lat in zip(heads, latents)]
    rows = sum(h.out_features for h in heads)
    flat = torch.empty(sum(h.generator.size for h in heads), dtype=kernel_dtype, device=latents[0].device)
    outs, off = [], 0
    for h in heads:
        outs.append(flat[off:off + h.generator.size])
        off += h.generator.size
    ops.materialize_weights(specs, outs)
    if layout == "rows":
        weight = flat.view(rows, heads[0].in_features)
    else:
        out_f, in_f = heads[0].out_features, heads[0].in_features
        weight = flat.view(len(heads), out_f, in_f).permute(1, 0, 2).reshape(out_f, len(heads) * in_f)
    return weight if kernel_dtype == dtype else weight.to(dtype=dtype)


class _HeadsLinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input, bias, heads, layout, *latents):
        with torch.no_grad():
            weight = _weight(heads, latents, input.dtype, layout)
        ctx.save_for_backward(input, *latents)
        ctx.heads = heads
        ctx.layout = layout
        ctx.has_bias = bias is not None
        return F.linear(input, weight, bias)

    @staticmethod
    def backward(ctx, grad_output):
        input, *latents = ctx.saved_tensors
        heads, layout = ctx.heads, ctx.layout
        out_total = grad_output.shape[-1]
        in_total = input.shape[-1]
        grad_2d = grad_output.reshape(-1, out_total)
        grad_input = grad_bias = None
        grad_latents = [None] * len(latents)
        if ctx.needs_input_grad[0]:
            with torch.no_grad():
                weight = _weight(heads, latents, grad_output.dtype, layout)
            grad_input = grad_2d.matmul(weight).reshape_as(input)
        if any(ctx.needs_input_grad[4:]):
            ldt = latents[0].dtype
            gw = grad_2d.to(dtype=ldt).t().matmul(input.reshape(-1, in_total).to(dtype=ldt))  # [out, in]
            pieces, off = [], 0
            for h in heads:
                if layout == "rows":
                    pieces.append(gw[off:off + h.out_features].reshape(-1))
                    off += h.out_features
                else:
                    pieces.append(gw[:, off:off + h.in_features].contiguous().reshape(-1))
                    off += h.in_features
            specs = [(lat, p, h.generator.size, h.generator.layers, h.generator.seed, h.weight_scale, None)
                     for lat, p, h in zip(latents, pieces, heads)]
            grad_latents = ops.flush_weight_grads(specs)
        if ctx.has_bias and ctx.needs_input_grad[1]:
            grad_bias = grad_2d.sum(dim=0).to(dtype=grad_output.dtype)
        return (grad_input, grad_bias, None, None, *grad_latents)


def block_fht_headwise_linear(input: torch.Tensor, heads: Sequence[BlockFHTLinear]) -> torch.Tensor:
    """``torch.cat([head(input) for head in heads], dim=-1)`` with every head's weight
    generated in one launch (``HeadwiseLinear.forward``, reference
    ``examples/nanogpt/model.py:160-175``; heads share ``in_features``)."""
    heads = list(heads)
    _native.require_cuda(input)
    biases = [h.bias for h in heads]
    uniform_bias = all(b is None for b in biases) or all(b is not None for b in biases)
    if (not uniform_bias or any(h.in_features != input.shape[-1] for h in heads)
            or not _batchable(heads, input.dtype)):
        return torch.cat([h(input) for h in heads], dim=-1)
    bias = None if biases[0] is None else torch.cat(biases, dim=0)
    return _HeadsLinearFn.apply(input, bias, heads, "rows", *[h.generator.latent for h in heads])


def block_fht_grouped_input_linear(input: torch.Tensor, heads: Sequence[BlockFHTLinear]) -> torch.Tensor:
    """``sum_i heads[i](piece_i)`` over equal splits of the last dimension, with every
    head's weight generated in one launch (``GroupedInputLinear.forward``, reference
    ``examples/nanogpt/model.py:272-277``; only the first head may carry a bias)."""
    heads = list(heads)
    _native.require_cuda(input)
    group = heads[0].in_features if heads else 0
    same_shape = all(h.in_features == group and h.out_features == heads[0].out_features for h in heads)
    if (not same_shape or group * len(heads) != input.shape[-1] or any(h.bias is not None for h in heads[1:])
            or not _batchable(heads, input.dtype)):
        pieces = input.split(group, dim=-1)
        out = heads[0](pieces[0])
        for piece, head in zip(pieces[1:], heads[1:]):
            out = out + head(piece)
        return out
    return _HeadsLinearFn.apply(input, heads[0].bias, heads, "cols", *[h.generator.latent for h in heads])
