"""Pins the CPU oracle before anything is checked against it.

Each check is chosen so that a plausible slip in the oracle (a wrong constant,
shift, bit order, sign order, normalization or index) fails it:

* golden vectors written from the reference's own CPU path
  (tests/golden/make_golden.py);
* closed forms and identities that fix the mathematics independently of the
  reference code (lowbias32's published inverse, the Sylvester Hadamard matrix,
  involution, orthogonality, adjointness, finite differences).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import decode_array
from oracle import c_oracle
from oracle import oracle as O


# ---------------------------------------------------------------- hash / signs

def lowbias32_inverse(x: int) -> int:
    """Published inverse of the lowbias32 hash (C. Wellons, hash-prospector):
    x ^= x>>16; x *= 0x43021123; x ^= x>>15 ^ x>>30; x *= 0x1d69e2a5; x ^= x>>16."""
    m = 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x43021123) & m
    x ^= (x >> 15) ^ (x >> 30)
    x = (x * 0x1D69E2A5) & m
    x ^= x >> 16
    return x


def test_lowbias32_is_inverted_by_published_inverse():
    rng = np.random.default_rng(0)
    for x in [0, 1, 2, 0xFFFFFFFF, 0x80000000] + [int(v) for v in rng.integers(0, 2**32, 2000)]:
        assert lowbias32_inverse(O.lowbias32(x)) == x
    assert O.lowbias32(0) == 0


def test_lowbias32_inverse_catches_wrong_constant():
    # A slip in a multiplier must break the identity (the pin is not vacuous).
    def bad(x):
        x ^= x >> 16
        x = (x * 0x7FEB352F) & 0xFFFFFFFF
        x ^= x >> 15
        x = (x * 0x846CA68B) & 0xFFFFFFFF
        x ^= x >> 16
        return x

    assert any(lowbias32_inverse(bad(x)) != x for x in range(1, 100))


def test_sign_words_match_reference_golden(golden):
    rows = golden["sign_words"]
    assert len(rows) > 1000
    for seed, block, layer, word, value in rows:
        assert O.sign_word_for(seed, block, layer, word) == value, (seed, block, layer, word)
        assert c_oracle.sign_word(seed, block, layer, word) == value, (seed, block, layer, word)


def test_vectorized_sign_words_match_scalar(golden):
    for seed in (0, -1, 2**63 - 1, -(2**63), 123):
        for block in (0, 7, 2**32 - 1):
            vec = O.sign_words(seed, block, 2, 300, first_word=5)
            cvec = c_oracle.sign_words(seed, block, 2, 300, first_word=5)
            assert np.array_equal(vec, cvec)
            assert all(int(vec[i]) == O.sign_word_for(seed, block, 2, 5 + i) for i in range(0, 300, 37))


def test_sign_vectors_match_reference_golden(golden):
    for case in golden["signs"]:
        got = O.sign_vector(case["seed"], case["block"], case["layer"], case["block_size"])
        assert got.tolist() == [float(v) for v in case["signs"]], case


def test_sign_bit_layout_port_of_reference_test():
    # tests/test_block_fht.py:25-31: position p uses bit p&31 of word p>>5.
    got = O.sign_vector(999, 3, 2, 65)
    expected = [1.0 if ((O.sign_word_for(999, 3, 2, p >> 5) >> (p & 31)) & 1) else -1.0 for p in range(65)]
    assert got.tolist() == expected


# ---------------------------------------------------------------- FHT

def sylvester(B: int) -> np.ndarray:
    idx = np.arange(B)
    pc = np.vectorize(lambda v: bin(int(v)).count("1"))(idx[:, None] & idx[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0) / math.sqrt(B)


@pytest.mark.parametrize("B", [1, 2, 4, 8, 32, 128, 1024])
def test_fht_equals_sylvester_closed_form(B):
    rng = np.random.default_rng(B)
    x = rng.standard_normal((3, B))
    H = sylvester(B)
    np.testing.assert_allclose(O.fht_normalized(x), x @ H.T, rtol=1e-12, atol=1e-12)


def test_fht_identities():
    rng = np.random.default_rng(1)
    B = 4096
    x = rng.standard_normal(B)
    y = O.fht_normalized(x)
    np.testing.assert_allclose(O.fht_normalized(y), x, atol=1e-12)          # involution
    assert abs(np.linalg.norm(y) - np.linalg.norm(x)) < 1e-9                 # Parseval
    delta = np.zeros(B); delta[37] = 1.0
    col = O.fht_normalized(delta)
    want = np.array([(-1.0) ** bin(37 & i).count("1") for i in range(B)]) / math.sqrt(B)
    np.testing.assert_allclose(col, want, atol=1e-15)                         # delta -> column
    const = O.fht_normalized(np.ones(B))
    e0 = np.zeros(B); e0[0] = math.sqrt(B)
    np.testing.assert_allclose(const, e0, atol=1e-9)                          # constant -> sqrt(B) e0


# ---------------------------------------------------------------- forward / backward

def _golden_grad(case):
    if "grad_sumsq" in case:
        return decode_array(case["grad_sumsq"]), 1
    return decode_array(case["grad_sumsq_sampled"]), case["grad_sumsq_stride"]


def test_forward_and_backward_match_reference_golden(golden):
    for case in golden["slices"]:
        latent = decode_array(case["latent"])
        want = decode_array(case["out"])
        args = (case["size"], case["layers"], case["seed"], case["start"], case["stop"])
        got = O.slice_forward(latent, *args)
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12, err_msg=case["name"])
        got_c = c_oracle.forward(latent, *args)
        np.testing.assert_allclose(got_c, want, rtol=1e-10, atol=1e-12, err_msg=case["name"])
        # golden gradient is d/dlatent of sum(y^2), i.e. the adjoint applied to 2*y
        grad = O.slice_backward(2.0 * want, latent.shape[0], *args)
        grad_c = c_oracle.backward(2.0 * want, latent.shape[0], *args)
        gw, stride = _golden_grad(case)
        np.testing.assert_allclose(grad[::stride], gw, rtol=1e-9, atol=1e-10, err_msg=case["name"])
        np.testing.assert_allclose(grad_c[::stride], gw, rtol=1e-9, atol=1e-10, err_msg=case["name"])
        if stride != 1:
            assert abs(grad.sum() - case["grad_sumsq_sum"]) < 1e-8 * max(1.0, abs(case["grad_sumsq_sum"]))
        if "full_sample_index" in case:
            full = c_oracle.forward(latent, case["size"], case["layers"], case["seed"], 0, case["size"])
            np.testing.assert_allclose(full[case["full_sample_index"]], case["full_sample_value"],
                                       rtol=1e-10, atol=1e-12)
            assert abs(full.sum() - case["full_sum"]) < 1e-8 * max(1.0, abs(case["full_sum"]))
            assert abs(np.square(full).sum() - case["full_sumsq"]) < 1e-9 * case["full_sumsq"]


def test_slice_equals_full_and_orthogonality():
    rng = np.random.default_rng(2)
    latent = rng.standard_normal(100)  # B = 128, zero padded
    full = O.slice_forward(latent, 1000, 3, 5, 0, 1000)
    np.testing.assert_allclose(O.slice_forward(latent, 1000, 3, 5, 129, 777), full[129:777], atol=0)
    # each generated block is an orthogonal image of the padded latent
    for b in range(7):
        assert abs(np.linalg.norm(full[b * 128:(b + 1) * 128]) - np.linalg.norm(latent)) < 1e-9


def test_adjoint_identity_and_finite_differences():
    rng = np.random.default_rng(3)
    n, size, L, seed, start, stop = 50, 700, 3, -17, 33, 611
    x = rng.standard_normal(n)
    g = rng.standard_normal(stop - start)
    y = O.slice_forward(x, size, L, seed, start, stop)
    xt = O.slice_backward(g, n, size, L, seed, start, stop)
    assert abs(np.dot(y, g) - np.dot(x, xt)) < 1e-9 * max(1.0, abs(np.dot(y, g)))
    # finite differences of <T x, g> along a random direction
    d = rng.standard_normal(n)
    eps = 1e-6
    fd = (np.dot(O.slice_forward(x + eps * d, size, L, seed, start, stop), g)
          - np.dot(O.slice_forward(x - eps * d, size, L, seed, start, stop), g)) / (2 * eps)
    assert abs(fd - np.dot(xt, d)) < 1e-6 * max(1.0, abs(fd))


def test_c_oracle_matches_numpy_oracle_multiblock():
    rng = np.random.default_rng(4)
    latent = rng.standard_normal(3000)  # B = 4096
    args = (50_000, 2, 2**40 + 1, 4000, 41_234)
    np.testing.assert_allclose(c_oracle.forward(latent, *args), O.slice_forward(latent, *args), atol=1e-12)
    g = rng.standard_normal(args[4] - args[3])
    np.testing.assert_allclose(c_oracle.backward(g, 3000, *args), O.slice_backward(g, 3000, *args),
                               atol=1e-10)


def test_invalid_slice_raises():
    with pytest.raises(ValueError):
        O.slice_forward(np.ones(4), 10, 1, 0, 5, 11)
    with pytest.raises(ValueError):
        c_oracle.forward(np.ones(4), 10, 1, 0, 6, 5)


# ---------------------------------------------------------------- linear

def test_linear_matches_reference_golden(golden):
    for case in golden["linear"]:
        latent = decode_array(case["latent"])
        x = decode_array(case["x"]).reshape(case["tokens"], case["in_features"])
        want = decode_array(case["out"]).reshape(case["tokens"], case["out_features"])
        got = O.linear_forward(x, latent, case["out_features"], case["layers"], case["seed"],
                               case["weight_scale"])
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- torch port

def test_torch_port_matches_oracle():
    import torch

    rng = np.random.default_rng(5)
    latent = rng.standard_normal(200)
    lat_t = torch.tensor(latent, dtype=torch.float64, requires_grad=True)
    y = O.torch_port_slice(lat_t, 1500, 3, 77, 255, 1290)
    np.testing.assert_allclose(y.detach().numpy(), O.slice_forward(latent, 1500, 3, 77, 255, 1290), atol=1e-12)
    y.square().sum().backward()
    want = O.slice_backward(2 * y.detach().numpy(), 200, 1500, 3, 77, 255, 1290)
    np.testing.assert_allclose(lat_t.grad.numpy(), want, atol=1e-10)


# ---------------------------------------------------------------- signed activation FHT

@pytest.mark.parametrize("features", [1, 5, 8, 100, 256])
def test_fixed_fht_mix_equals_dense_signed_hadamard(features):
    rng = np.random.default_rng(features)
    P = O.next_power_of_two(features)
    signs = rng.integers(0, 2, P) * 2.0 - 1.0
    x = rng.standard_normal((4, features))
    M = np.diag(signs) @ sylvester(P) @ np.diag(signs)
    xp = np.zeros((4, P))
    xp[:, :features] = x
    want = (xp @ M.T)[:, :features]
    np.testing.assert_allclose(O.fixed_fht_mix(x, signs), want, rtol=1e-12, atol=1e-12)


def test_fixed_fht_mix_involution_and_parseval():
    rng = np.random.default_rng(3)
    signs = rng.integers(0, 2, 1024) * 2.0 - 1.0
    x = rng.standard_normal((3, 1024))
    y = O.fixed_fht_mix(x, signs)
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-12)
    np.testing.assert_allclose(O.fixed_fht_mix(y, signs), x, rtol=1e-10, atol=1e-12)
    # a single sign multiply is not an involution: the check would catch that mistake
    once = O.fht_normalized(x * signs)
    assert np.abs(O.fht_normalized(once * signs) - x).max() > 1e-3
