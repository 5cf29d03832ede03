"""CPU oracle for the BlockFHT path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for the
baseline, as the thing timed on the host).  The product package
``latent_weight_lab_amd`` never imports it and has no CPU fallback.

It restates, in numpy, the semantics of the reference path:

* ``lowbias32`` / ``sign_word_for``  — ``latent_weight_lab/block_fht.py:36-52``
  (device twin ``csrc/block_fht_ext_cuda.cu:27-43``)
* ``sign_vector``                    — ``block_fht.py:55-81`` (``signs_for``)
* ``fht_normalized``                 — ``block_fht.py:18-33``
* ``slice_forward``                  — ``block_fht.py:84-109`` (``block_fht_slice_torch``)
* ``slice_backward``                 — the adjoint that ``block_fht.py:180-196`` obtains
  by autograd and ``block_fht_ext_cuda.cu:185-223`` computes explicitly
* ``linear_forward``                 — ``block_fht.py:251-288`` fallback branch
* ``fixed_fht_mix``                  — ``examples/nanogpt/model.py:200-218`` (``FixedFHTMix``)

and, for the CPU baseline, ``torch_port_slice`` — an op-for-op restatement of
``block_fht_slice_torch`` in torch CPU ops (per-block Python loop, reshape
butterflies, vectorized int64 hash), differentiable by autograd like the
reference's fallback.

How each function is pinned (tests/test_oracle.py):

* ``lowbias32``: composed with the independently published inverse of the
  lowbias32 hash it must give the identity on random words, and it must agree
  with the reference's golden words.
* ``sign_word_for`` / ``sign_vector``: the reference's golden vectors
  (``tests/golden/bfht_golden.json``, written from the reference by
  ``tests/golden/make_golden.py``).
* ``fht_normalized``: the closed form ``H[i, j] = (-1)^popcount(i & j) / sqrt(B)``
  (dense brute force), involution, Parseval, delta and constant inputs.
* ``slice_forward`` / ``slice_backward``: golden vectors, adjoint identity,
  finite differences, slice == full[start:stop].
* ``linear_forward``: golden vectors, and equality with a dense matmul on the
  materialized weight.
* ``fixed_fht_mix``: the dense product ``diag(s) H diag(s)`` with the closed-form
  H on the padded input, involution and Parseval at power-of-two widths.
"""
from __future__ import annotations

import math

import numpy as np

MASK32 = 0xFFFFFFFF
GOLDEN_BLOCK = 0x9E3779B9
GOLDEN_LAYER = 0x85EBCA6B
GOLDEN_WORD = 0xC2B2AE35


def next_power_of_two(value: int) -> int:
    """``block_fht.py:12-15``."""
    if value <= 0:
        raise ValueError("value must be positive")
    return 1 << (int(value) - 1).bit_length()


def lowbias32(x: int) -> int:
    """Scalar avalanche hash, ``block_fht.py:36-43``."""
    x &= MASK32
    x ^= x >> 16
    x = (x * 0x7FEB352D) & MASK32
    x ^= x >> 15
    x = (x * 0x846CA68B) & MASK32
    x ^= x >> 16
    return x


def seed32(seed: int) -> int:
    """Fold an int64 seed to 32 bits; Python's ``>>`` is arithmetic like the
    reference (``block_fht.py:47``)."""
    return (int(seed) ^ (int(seed) >> 32)) & MASK32


def sign_word_for(seed: int, block: int, layer: int, word: int) -> int:
    """``block_fht.py:46-52``."""
    x = seed32(seed)
    x ^= (GOLDEN_BLOCK * (int(block) + 1)) & MASK32
    x ^= (GOLDEN_LAYER * (int(layer) + 1)) & MASK32
    x ^= (GOLDEN_WORD * (int(word) + 1)) & MASK32
    return lowbias32(x)


def sign_words(seed: int, block: int, layer: int, nwords: int, first_word: int = 0) -> np.ndarray:
    """Vectorized ``sign_word_for`` over words ``first_word .. first_word+nwords``.

    uint32 numpy arithmetic wraps mod 2^32 exactly as the reference's masked
    int64 arithmetic does (``block_fht.py:67-78``).
    """
    w = np.arange(first_word, first_word + nwords, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = np.full(nwords, seed32(seed), dtype=np.uint32)
        x ^= np.uint32((GOLDEN_BLOCK * (int(block) + 1)) & MASK32)
        x ^= np.uint32((GOLDEN_LAYER * (int(layer) + 1)) & MASK32)
        x ^= ((np.uint64(GOLDEN_WORD) * (w + np.uint64(1))) & np.uint64(MASK32)).astype(np.uint32)
        x ^= x >> np.uint32(16)
        x *= np.uint32(0x7FEB352D)
        x ^= x >> np.uint32(15)
        x *= np.uint32(0x846CA68B)
        x ^= x >> np.uint32(16)
    return x


def sign_vector(seed: int, block: int, layer: int, block_size: int, dtype=np.float64) -> np.ndarray:
    """``signs_for`` (``block_fht.py:55-81``): bit ``p & 31`` of word ``p >> 5``;
    a set bit is +1, a clear bit is -1."""
    words = sign_words(seed, block, layer, (block_size + 31) // 32)
    bits = (words[:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & np.uint32(1)
    return (2.0 * bits.reshape(-1)[:block_size].astype(dtype) - 1.0).astype(dtype)


def fht_normalized(values: np.ndarray) -> np.ndarray:
    """Sylvester-ordered Walsh-Hadamard transform along the last axis, divided
    by sqrt(size) (``block_fht.py:18-33``): stage ``step`` pairs (a, a+step)."""
    size = values.shape[-1]
    if size <= 0 or size & (size - 1):
        raise ValueError("FHT size must be a positive power of two")
    out = np.array(values, copy=True)
    lead = out.shape[:-1]
    step = 1
    while step < size:
        v = out.reshape(*lead, -1, 2, step)
        first = v[..., 0, :].copy()
        second = v[..., 1, :].copy()
        v[..., 0, :] = first + second
        v[..., 1, :] = first - second
        out = v.reshape(*lead, size)
        step *= 2
    return out / out.dtype.type(math.sqrt(size))


def block_transform(latent: np.ndarray, block: int, layers: int, seed: int, dtype=np.float64) -> np.ndarray:
    """One generated block: ``D_L H ... D_1 H D_0 pad(latent)`` (``block_fht.py:98-107``)."""
    n = latent.shape[0]
    B = next_power_of_two(n)
    v = np.zeros(B, dtype=dtype)
    v[:n] = latent.astype(dtype)
    v = v * sign_vector(seed, block, 0, B, dtype)
    for layer in range(layers):
        v = fht_normalized(v)
        v = v * sign_vector(seed, block, layer + 1, B, dtype)
    return v


def check_slice(size: int, start: int, stop: int) -> None:
    if not 0 <= start <= stop <= size:
        raise ValueError(f"invalid slice [{start}, {stop}) for size {size}")


def slice_forward(latent: np.ndarray, size: int, layers: int, seed: int, start: int, stop: int,
                  dtype=np.float64) -> np.ndarray:
    """``block_fht_slice_torch`` (``block_fht.py:84-109``)."""
    check_slice(size, start, stop)
    B = next_power_of_two(latent.shape[0])
    pieces = []
    for block in range(start // B, (stop + B - 1) // B):
        lo = max(start - block * B, 0)
        hi = min(stop - block * B, B)
        pieces.append(block_transform(latent, block, layers, seed, dtype)[lo:hi])
    return np.concatenate(pieces) if pieces else np.zeros(0, dtype=dtype)


def slice_backward(grad_out: np.ndarray, latent_size: int, size: int, layers: int, seed: int,
                   start: int, stop: int, dtype=np.float64) -> np.ndarray:
    """Adjoint of ``slice_forward``: for each block, scatter the gradient into
    the block frame and apply ``D_0 H D_1 ... H D_L`` (H is symmetric, D
    diagonal), then sum the first ``latent_size`` entries over blocks."""
    check_slice(size, start, stop)
    B = next_power_of_two(latent_size)
    grad = np.zeros(latent_size, dtype=dtype)
    for block in range(start // B, (stop + B - 1) // B):
        lo = max(start - block * B, 0)
        hi = min(stop - block * B, B)
        g = np.zeros(B, dtype=dtype)
        off = block * B + lo - start
        g[lo:hi] = grad_out[off:off + (hi - lo)]
        for layer in range(layers - 1, -1, -1):
            g = g * sign_vector(seed, block, layer + 1, B, dtype)
            g = fht_normalized(g)
        g = g * sign_vector(seed, block, 0, B, dtype)
        grad += g[:latent_size]
    return grad


def materialize_weight(latent: np.ndarray, in_features: int, out_features: int, layers: int,
                       seed: int, dtype=np.float64) -> np.ndarray:
    size = in_features * out_features
    return slice_forward(latent, size, layers, seed, 0, size, dtype).reshape(out_features, in_features)


def linear_forward(x: np.ndarray, latent: np.ndarray, out_features: int, layers: int, seed: int,
                   weight_scale: float = 1.0, dtype=np.float64) -> np.ndarray:
    """``block_fht_linear_forward`` fallback (``block_fht.py:282-288``):
    ``out = x @ (weight_scale * W)^T`` with ``W = flat.view(out, in)``."""
    in_features = x.shape[-1]
    w = materialize_weight(latent, in_features, out_features, layers, seed, dtype) * dtype(weight_scale)
    flat = x.reshape(-1, in_features).astype(dtype)
    return (flat @ w.T).reshape(*x.shape[:-1], out_features)


def fixed_fht_mix(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``FixedFHTMix.forward`` (``examples/nanogpt/model.py:200-218``): zero-pad the
    last dimension to ``P = next_power_of_two(features)``, multiply by the ±1
    ``signs`` [P], ``normalized_fht_last_dim`` (``model.py:180-197``, the same
    transform as ``fht_normalized``), multiply by ``signs`` again, keep the first
    ``features`` values."""
    features = x.shape[-1]
    padded = next_power_of_two(features)
    xp = np.zeros(x.shape[:-1] + (padded,), dtype=np.float64)
    xp[..., :features] = x
    y = fht_normalized(xp * signs) * signs
    return y[..., :features]


def rel_l2(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = float(np.linalg.norm(want))
    num = float(np.linalg.norm(got - want))
    return num / den if den > 0 else num


# --------------------------------------------------------------------------
# torch CPU port: the reference's fallback algorithm, op for op, used as the
# timed CPU baseline (it is what a reference user without the GPU extension
# runs).  Imported lazily so the numpy oracle does not need torch.
# --------------------------------------------------------------------------

def _torch_signs(reference, block: int, layer: int, seed: int, block_size: int):
    import torch

    words = torch.arange((block_size + 31) // 32, device=reference.device, dtype=torch.int64)
    mixed = torch.full_like(words, seed32(seed))
    mixed = mixed ^ ((GOLDEN_BLOCK * (block + 1)) & MASK32)
    mixed = mixed ^ ((GOLDEN_LAYER * (layer + 1)) & MASK32)
    mixed = (mixed ^ ((GOLDEN_WORD * (words + 1)) & MASK32)) & MASK32
    mixed = (mixed ^ (mixed >> 16)) & MASK32
    mixed = (mixed * 0x7FEB352D) & MASK32
    mixed = (mixed ^ (mixed >> 15)) & MASK32
    mixed = (mixed * 0x846CA68B) & MASK32
    mixed = (mixed ^ (mixed >> 16)) & MASK32
    bits = (mixed.unsqueeze(1) >> torch.arange(32, dtype=torch.int64)) & 1
    return (2.0 * bits.reshape(-1)[:block_size] - 1.0).to(dtype=reference.dtype)


def _torch_fht(values):
    size = values.shape[-1]
    out = values.clone()
    step = 1
    while step < size:
        shape = out.shape
        out = out.reshape(*shape[:-1], -1, 2, step)
        first = out[..., 0, :].clone()
        second = out[..., 1, :].clone()
        out[..., 0, :] = first + second
        out[..., 1, :] = first - second
        out = out.reshape(shape)
        step *= 2
    return out / math.sqrt(size)


def torch_port_slice(latent, size: int, layers: int, seed: int, start: int, stop: int):
    """Op-for-op port of ``block_fht_slice_torch`` (``block_fht.py:84-109``)."""
    check_slice(size, start, stop)
    block_size = next_power_of_two(latent.numel())
    pieces = []
    for block in range(start // block_size, (stop + block_size - 1) // block_size):
        lo = max(start - block * block_size, 0)
        hi = min(stop - block * block_size, block_size)
        values = latent.new_zeros(block_size)
        values[: latent.numel()] = latent
        values = values * _torch_signs(latent, block, 0, seed, block_size)
        for layer in range(layers):
            values = _torch_fht(values)
            values = values * _torch_signs(latent, block, layer + 1, seed, block_size)
        pieces.append(values[lo:hi])
    import torch

    return torch.cat(pieces) if pieces else latent.new_empty(0)
