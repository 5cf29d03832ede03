"""latent_weight_lab_amd — the BlockFHT path of latent-weight-lab on MI355X.

Public names follow the reference package ``latent_weight_lab``
(``latent_weight_lab/__init__.py:1-23``).  The generator, its backward and the
fused linear run in hand-written gfx950 HIP kernels (``csrc/``) behind the C
ABI declared in ``include/lwl_bfht.h``.
"""
from .block_fht import (
    BlockFHT,
    BlockFHTLinear,
    block_fht_grad_latent,
    block_fht_linear_forward,
    block_fht_slice,
    flush_block_fht_weight_cache,
    forward_fused_grouped,
    lowbias32,
    next_power_of_two,
    prepare_block_fht_weight_cache,
    restore_block_fht_weight_cache,
    sign_word_for,
    signs_for,
    suspend_block_fht_weight_cache,
)
from .batched import block_fht_grouped_input_linear, block_fht_headwise_linear
from .mix import FixedFHTMix, fixed_fht_mix

__all__ = [
    "BlockFHT",
    "BlockFHTLinear",
    "FixedFHTMix",
    "block_fht_grad_latent",
    "block_fht_grouped_input_linear",
    "block_fht_headwise_linear",
    "block_fht_linear_forward",
    "block_fht_slice",
    "fixed_fht_mix",
    "flush_block_fht_weight_cache",
    "forward_fused_grouped",
    "lowbias32",
    "next_power_of_two",
    "prepare_block_fht_weight_cache",
    "restore_block_fht_weight_cache",
    "sign_word_for",
    "signs_for",
    "suspend_block_fht_weight_cache",
]
