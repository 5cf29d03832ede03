"""Fixed signed Walsh-Hadamard mixing of activations (the nanoGPT example's
``FixedFHTMix``, reference ``examples/nanogpt/model.py:200-218``): pad the last
dimension to a power of two, multiply by a fixed ±1 buffer, apply the normalized
Sylvester FHT, multiply by the buffer again, keep the original width.

The reference runs ``normalized_fht_last_dim`` (``model.py:180-197``) as a torch
loop of log2(P) reshape / clone stages in the activation dtype; here one HIP
launch does the whole row transform (``lwl_fht_mix``): in float32 with one
rounding, or for bfloat16 / float16 rows of 1024 and 4096 values (GPT-2's 768
and 3072 features) on the matrix cores, with one intermediate rounding to the
activation dtype between its two radix-32 stages.  The map is symmetric, so its
backward is the same launch on the gradient.
"""
from __future__ import annotations

import torch
from torch import nn

from . import ops


class _FHTMixFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, signs):
        ctx.save_for_backward(signs)
        return ops.fht_mix(x, signs)

    @staticmethod
    def backward(ctx, grad):
        (signs,) = ctx.saved_tensors
        return ops.fht_mix(grad.contiguous(), signs), None


def fixed_fht_mix(x: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """``(S H S pad(x))[..., :features]``, differentiable in ``x``."""
    return _FHTMixFn.apply(x, signs)


class FixedFHTMix(nn.Module):
    """Same constructor, buffer and forward contract as the reference module
    (``model.py:200-218``); the sign buffer is drawn exactly as there, from a CPU
    generator seeded with ``seed``."""

    def __init__(self, features: int, seed: int) -> None:
        super().__init__()
        self.features = int(features)
        self.padded = ops.next_power_of_two(self.features)
        generator = torch.Generator(device="cpu")
        generator.manual_seed(int(seed))
        signs = torch.randint(0, 2, (self.padded,), generator=generator, dtype=torch.float32) * 2.0 - 1.0
        self.register_buffer("signs", signs, persistent=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.features:
            raise ValueError(f"expected last dim {self.features}, got {x.shape[-1]}")
        return fixed_fht_mix(x, self.signs.to(device=x.device))
