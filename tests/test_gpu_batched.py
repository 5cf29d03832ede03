"""GPU parity of the batched multi-head linears (one grouped generation for all heads):
``block_fht_headwise_linear`` against ``torch.cat([head(x) ...])`` and
``block_fht_grouped_input_linear`` against ``sum(head(piece))`` — the nanoGPT
example's HeadwiseLinear / GroupedInputLinear (reference
``examples/nanogpt/model.py:136-175,241-277``) evaluated head by head.

The generated weights are bit-identical to the per-head ones; outputs and
gradients go through GEMMs of other shapes (all heads at once), so they are
compared within float32 rounding (1e-5 relative L2) — and bf16 activations within
the bf16 bar (1e-2) — and every head's latent gradient against the C oracle.
"""
from __future__ import annotations

import copy

import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import BlockFHTLinear, block_fht_grouped_input_linear, block_fht_headwise_linear
from latent_weight_lab_amd.batched import _weight
from latent_weight_lab_amd.block_fht import _generated_weight
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def rel(a, b):
    return O.rel_l2(a.detach().double().cpu().numpy().reshape(-1), b.detach().double().cpu().numpy().reshape(-1))


def make_heads(n, in_f, out_f, bias, **kw):
    torch.manual_seed(n + in_f + out_f)
    heads = [BlockFHTLinear(in_f, out_f, bias=bias, latent_ratio=0.01, layers=2, seed=1000 + 64 * 3 + i, **kw)
             for i in range(n)]
    for h in heads:
        if h.bias is not None:
            torch.nn.init.normal_(h.bias, std=0.1)
    return [h.cuda() for h in heads]


def run(fn, heads, x, g):
    for h in heads:
        h.zero_grad(set_to_none=True)
    x = x.detach().clone().requires_grad_(True)
    y = fn(x, heads)
    (y.float() * g).sum().backward()
    return y.detach(), x.grad, [h.generator.latent.grad.clone() for h in heads], \
        [None if h.bias is None else h.bias.grad.clone() for h in heads]


def per_head_cat(x, heads):
    return torch.cat([h(x) for h in heads], dim=-1)


def per_head_sum(x, heads):
    pieces = x.split(heads[0].in_features, dim=-1)
    out = heads[0](pieces[0])
    for p, h in zip(pieces[1:], heads[1:]):
        out = out + h(p)
    return out


@pytest.mark.parametrize("bias", [False, True])
def test_headwise_matches_per_head(bias):
    # GPT-2-small attention heads: 12 x (768 -> 64), latent 492 (block 2^9)
    heads = make_heads(12, 768, 64, bias)
    x = torch.randn(3, 50, 768, device="cuda")
    g = torch.randn(3, 50, 12 * 64, device="cuda")
    y, gx, gl, gb = run(block_fht_headwise_linear, heads, x, g)
    y2, gx2, gl2, gb2 = run(per_head_cat, heads, x, g)
    assert y.shape == y2.shape
    assert rel(y, y2) < 1e-5
    assert rel(gx, gx2) < 1e-5
    for a, b in zip(gl, gl2):
        assert rel(a, b) < 1e-5
    if bias:
        for a, b in zip(gb, gb2):
            assert rel(a, b) < 1e-5


def test_headwise_weight_is_per_head_weight_bitwise():
    heads = make_heads(5, 96, 40, False)
    lats = [h.generator.latent for h in heads]
    for dtype in (torch.float32, torch.bfloat16):
        w = _weight(heads, lats, dtype, "rows")
        want = torch.cat([_generated_weight(h.generator.latent, h.generator.size, 2, h.generator.seed,
                                            h.weight_scale, 0.0).view(40, 96).to(dtype) for h in heads])
        assert torch.equal(w, want)


def test_headwise_latent_grads_match_oracle():
    heads = make_heads(4, 128, 32, False)
    x = torch.randn(40, 128, device="cuda")
    g = torch.randn(40, 4 * 32, device="cuda")
    _, _, gl, _ = run(block_fht_headwise_linear, heads, x, g)
    gw_all = g.double().cpu().numpy().T @ x.double().cpu().numpy()
    for i, (h, got) in enumerate(zip(heads, gl)):
        gw = gw_all[32 * i:32 * (i + 1)]
        want = h.weight_scale * c_oracle.backward(gw.reshape(-1), h.generator.latent.numel(), h.generator.size, 2,
                                                  h.generator.seed, 0, h.generator.size)
        assert O.rel_l2(got.double().cpu().numpy(), want) < 1e-5


def test_headwise_bf16_activations():
    heads = make_heads(12, 768, 64, False)
    x = torch.randn(2, 64, 768, device="cuda").to(torch.bfloat16)
    g = torch.randn(2, 64, 768, device="cuda")
    y, gx, gl, _ = run(block_fht_headwise_linear, heads, x, g)
    y2, gx2, gl2, _ = run(per_head_cat, heads, x, g)
    assert y.dtype == torch.bfloat16
    assert rel(y, y2) < 1e-2 and rel(gx, gx2) < 1e-2
    for a, b in zip(gl, gl2):
        assert rel(a, b) < 1e-5  # grad_weight in the fp32 latent dtype on both paths


@pytest.mark.parametrize("bias", [False, True])
def test_grouped_input_matches_per_head(bias):
    # c_proj split into 4 input groups: 4 x (768 -> 768), latent 5898 (block 2^13); bias on head 0
    heads = make_heads(4, 768, 768, False)
    if bias:
        heads[0].bias = torch.nn.Parameter(torch.randn(768, device="cuda") * 0.1)
    x = torch.randn(2, 30, 4 * 768, device="cuda")
    g = torch.randn(2, 30, 768, device="cuda")
    y, gx, gl, gb = run(block_fht_grouped_input_linear, heads, x, g)
    y2, gx2, gl2, gb2 = run(per_head_sum, heads, x, g)
    assert rel(y, y2) < 1e-5 and rel(gx, gx2) < 1e-5
    for a, b in zip(gl, gl2):
        assert rel(a, b) < 1e-5
    if bias:
        assert rel(gb[0], gb2[0]) < 1e-5


def test_heads_with_gains_run_head_by_head():
    heads = make_heads(3, 64, 32, False, output_gain=True)
    x = torch.randn(10, 64, device="cuda")
    g = torch.randn(10, 96, device="cuda")
    y, gx, gl, _ = run(block_fht_headwise_linear, heads, x, g)
    y2, gx2, gl2, _ = run(per_head_cat, heads, x, g)
    assert torch.equal(y, y2) and torch.equal(gx, gx2)
    for a, b in zip(gl, gl2):
        assert torch.equal(a, b)


def test_cached_heads_use_the_cache():
    # with a live cache the heads' cached weights are used, as HeadwiseLinear does
    from latent_weight_lab_amd import flush_block_fht_weight_cache, prepare_block_fht_weight_cache

    heads = make_heads(3, 64, 32, False)
    model = torch.nn.ModuleList(heads)
    ref = copy.deepcopy(model)
    prepare_block_fht_weight_cache(model)
    x = torch.randn(10, 64, device="cuda")
    y = block_fht_headwise_linear(x, list(model))
    y2 = per_head_cat(x, list(ref))
    assert rel(y, y2) < 1e-6
    y.sum().backward()
    flush_block_fht_weight_cache(model)
    y2.sum().backward()
    for a, b in zip(model, ref):
        assert rel(a.generator.latent.grad, b.generator.latent.grad) < 1e-5
