"""GPU parity of BlockFHTLinear's forward (reference latent_weight_lab/block_fht.py:251-288).

The fused kernel (bf16, block 2^15: weights generated on chip and contracted on
MFMA, never materialized) and the generate + F.linear path for other shapes are
checked against float64 products with the weight the C oracle generates from the
same (bf16-rounded) latent.  Bar: bf16 1e-2 relative L2,
float32 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import decode_array, gpu_available
from latent_weight_lab_amd import BlockFHTLinear, block_fht_grad_latent, block_fht_linear_forward, block_fht_slice
from latent_weight_lab_amd import ops
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def oracle_linear(x: torch.Tensor, latent: torch.Tensor, out_f: int, layers: int, seed: int, scale: float):
    in_f = x.shape[-1]
    w = c_oracle.forward(latent.double().cpu().numpy(), in_f * out_f, layers, seed, 0, in_f * out_f)
    w = w.reshape(out_f, in_f)
    xf = x.reshape(-1, in_f).double().cpu().numpy()
    return (xf @ w.T) * scale


@pytest.mark.parametrize(
    "tokens,in_f,out_f,n,layers,seed,scale",
    [
        (4096, 768, 3072, 32768, 3, 3, 1.0),    # config 4, GPT-2 MLP up
        (4096, 3072, 768, 32768, 3, 3, 1.0),    # config 4, GPT-2 MLP down
        (17, 768, 2304, 32768, 3, 100, 0.5),    # qkv shape, ragged tokens
        (1, 768, 768, 32768, 2, 101, 2.0),      # decode batch 1, proj shape
        (64, 1024, 100, 20000, 1, -7, 1.0),     # in divides 2^15; last block partial; latent padded
        (33, 2048, 40, 32768, 3, 9, 0.25),      # rows of 2048 (16 per block)
        (300, 1000, 77, 30000, 2, 5, 1.0),      # in % 16 != 0, rows straddle blocks; tiled x, padded
        (255, 1024, 200, 32768, 2, 21, 1.0),    # just below the tiled-x batch size: x read in place
        (257, 1024, 200, 32768, 2, 21, 1.0),    # just above it: tiled x, last tile holds one token
        (20, 528, 200, 32768, 3, 31, 1.0),      # smallest in_features: 4 row tiles per block
        (40, 5120, 30, 32768, 2, 32, 1.0),      # largest: the k-major table fills all 160 KiB of LDS
        (333, 2048, 90, 32768, 3, 33, 1.0),     # two blocks per workgroup, exact table pitch (33 rows)
        (280, 1064, 90, 32768, 2, 36, 1.0),     # 32 rows per block: two blocks in 64-row tiles
        (320, 704, 64, 32768, 3, 37, 1.0),      # two blocks of 47 rows (6 row tiles), one token tile per workgroup
        (6144, 768, 3072, 32768, 3, 38, 1.0),   # two blocks per workgroup, 55 token tiles: one full round + 3 singles
        (600, 3072, 100, 32768, 2, 34, 0.5),    # two blocks per workgroup, 23-row pitch, 5 tiles
        (300, 5120, 41, 32768, 3, 35, 1.0),     # two blocks per workgroup, one row tile, last tile single
        # rows of 768: tiles of 64 whole rows (1.5 blocks, inside two generated blocks), no straddling rows
        (300, 768, 1000, 32768, 2, 39, 1.0),    # 16 row tiles, the last of 40 rows; ragged token tiles
        (513, 768, 2304, 32768, 3, 40, 0.5),    # GPT-2 qkv at a prefill batch: 36 tiles, one-token last tile
        (256, 768, 768, 20000, 1, 41, 1.0),     # GPT-2 proj, padded latent (last generated block partial)
        # rows of 3072 from 2048 tokens: tiles of three whole blocks (32 rows), the last 20 k steps'
        # W tiles read from the workgroup's overflow in global memory
        (2048, 3072, 700, 32768, 2, 42, 0.5),   # the smallest such batch; last tile 28 rows, its third block partial
        (3100, 3072, 40, 20000, 1, 43, 1.0),    # one layer, padded latent, ragged token tiles, last tile 8 rows
        (5000, 3072, 96, 32768, 3, 44, 1.0),    # three whole tiles, two rounds of token tiles
        (2047, 3072, 96, 32768, 3, 44, 1.0),    # just below it: two-block tiles with straddling rows
    ],
)
def test_fused_linear_matches_oracle(tokens, in_f, out_f, n, layers, seed, scale):
    g = torch.Generator().manual_seed(tokens + in_f)
    latent = torch.randn(n, generator=g).to(torch.bfloat16)
    x = torch.randn(tokens, in_f, generator=g).to(torch.bfloat16)
    xd, ld = x.cuda(), latent.cuda()
    assert ops.linear_supported(in_f, out_f, ld, xd), "fused kernel should take this shape"
    got = block_fht_linear_forward(xd, ld, out_f, layers, seed, weight_scale=scale, fused=True)
    torch.cuda.synchronize()
    assert got.shape == (tokens, out_f) and got.dtype == torch.bfloat16
    want = oracle_linear(x, latent, out_f, layers, seed, scale)
    err = O.rel_l2(got.double().cpu().numpy(), want)
    assert err < 1e-2, err
    # deterministic: no atomics, the straddling rows are summed in a fixed order
    again = block_fht_linear_forward(xd, ld, out_f, layers, seed, weight_scale=scale, fused=True)
    assert torch.equal(got, again)
    # the generate-once route (then a GEMM) agrees within the bf16 bar
    gen = block_fht_linear_forward(xd, ld, out_f, layers, seed, weight_scale=scale, fused=False)
    assert O.rel_l2(gen.double().cpu().numpy(), want) < 1e-2


def test_fused_linear_3d_input_and_module():
    torch.manual_seed(0)
    lin = BlockFHTLinear(768, 3072, latent_dim=32768, layers=3, seed=11).cuda().to(torch.bfloat16)
    x = torch.randn(2, 5, 768, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        fused = lin.forward_fused(x)
        dense = torch.nn.functional.linear(x.float(), lin.weight.float())
    assert fused.shape == (2, 5, 3072)
    assert O.rel_l2(fused.double().cpu().numpy(), dense.double().cpu().numpy()) < 1e-2


@pytest.mark.parametrize("dtype,n,in_f,out_f,layers,small,large", [
    (torch.bfloat16, 32768, 768, 3072, 3, 127, 128),   # block-2^15 kernel: fused below 128 tokens
    (torch.float16, 16384, 1024, 4096, 2, 7, 8),        # the reference's domain: fused below 8
])
def test_default_route_by_batch(dtype, n, in_f, out_f, layers, small, large):
    # the default route is the fused kernel for small batches and W generated once + GEMM from
    # the crossover on, bit for bit the same as asking for that route; forward_fused follows it
    g = torch.Generator().manual_seed(12)
    latent = torch.randn(n, generator=g).to(dtype).cuda()
    lin = BlockFHTLinear(in_f, out_f, bias=True, latent_dim=n, layers=layers, seed=6).cuda().to(dtype)
    with torch.no_grad():
        lin.generator.latent.copy_(latent)
        lin.bias.normal_()
    for tokens, fused in ((small, True), (large, False)):
        x = torch.randn(tokens, in_f, generator=g).to(dtype).cuda()
        assert ops.linear_supported(in_f, out_f, latent, x)
        assert ops.linear_fused_preferred(in_f, out_f, latent, x) == fused
        with torch.no_grad():
            auto = block_fht_linear_forward(x, latent, out_f, layers, 6)
            want = block_fht_linear_forward(x, latent, out_f, layers, 6, fused=fused)
            assert torch.equal(auto, want), (tokens, fused)
            mod = lin.forward_fused(x)
            if fused:
                ref = ops.linear_forward(x, latent, out_f, layers, 6, 1.0, bias=lin.bias)
            else:
                w = block_fht_slice(latent, in_f * out_f, layers, 6, 0, in_f * out_f).view(out_f, in_f)
                ref = torch.nn.functional.linear(x, w, lin.bias)
            assert torch.equal(mod, ref), (tokens, fused)


def test_generate_route_bitwise():
    # generate + GEMM: W equals the slice forward times weight_scale, rounded as the
    # reference's fallback (bf16 * scale in bf16), and the product is F.linear's
    g = torch.Generator().manual_seed(8)
    latent = torch.randn(32768, generator=g).to(torch.bfloat16).cuda()
    x = torch.randn(37, 768, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        got = block_fht_linear_forward(x, latent, 2304, 3, 5, weight_scale=0.5, fused=False)
        w = block_fht_slice(latent, 768 * 2304, 3, 5, 0, 768 * 2304).view(2304, 768) * 0.5
        want = torch.nn.functional.linear(x, w)
    assert torch.equal(got, want)


def test_generate_route_is_differentiable_in_the_latent():
    latent = torch.randn(4096, device="cuda", requires_grad=True)
    x = torch.randn(5, 64, device="cuda", requires_grad=True)
    y = block_fht_linear_forward(x, latent, 48, 2, 13, weight_scale=0.5)
    y.square().sum().backward()
    assert latent.grad is not None and x.grad is not None
    w = block_fht_slice(latent.detach(), 64 * 48, 2, 13, 0, 64 * 48).view(48, 64) * 0.5
    gy = 2 * (x.detach() @ w.t())
    want = 0.5 * block_fht_grad_latent(latent.detach(), (gy.t() @ x.detach()).reshape(-1), 64 * 48, 2, 13)
    assert O.rel_l2(latent.grad.double().cpu().numpy(), want.double().cpu().numpy()) < 1e-5


def test_unsupported_shapes_fall_back_to_generated_weight():
    # outside both fused kernels (here fp32, block 2^12, 4096 % 48 != 0) W is generated and
    # F.linear runs, as the reference's fallback (gate block_fht.py:263-273)
    g = torch.Generator().manual_seed(4)
    latent = torch.randn(4096, generator=g).cuda()
    x = torch.randn(9, 48, generator=g).cuda()
    assert not ops.linear_supported(48, 64, latent, x)
    got = block_fht_linear_forward(x, latent, 64, 2, 13, weight_scale=0.5)
    want = oracle_linear(x.cpu(), latent.cpu(), 64, 2, 13, 0.5)
    assert O.rel_l2(got.double().cpu().numpy(), want) < 1e-5


def test_linear_golden_vectors(golden):
    for case in golden["linear"]:
        latent = torch.tensor(decode_array(case["latent"]), dtype=torch.float32, device="cuda")
        x = torch.tensor(decode_array(case["x"]), dtype=torch.float32, device="cuda").reshape(
            case["tokens"], case["in_features"])
        got = block_fht_linear_forward(x, latent, case["out_features"], case["layers"], case["seed"],
                                       weight_scale=case["weight_scale"])
        want = decode_array(case["out"])
        assert O.rel_l2(got.double().cpu().numpy().reshape(-1), want) < 1e-5


@pytest.mark.parametrize("opts", [
    dict(bias=True),
    dict(bias=True, modulation_alpha=0.3),
    dict(bias=True, residual_base_scale=0.5),
    dict(bias=False, output_gain=True, input_gain=True),
])
def test_forward_fused_matches_materialized(opts):
    # reference tests/test_block_fht.py:196-199 and tests/test_block_fht_cuda.py:43-98:
    # forward_fused == F.linear(x, weight, bias) for every option
    torch.manual_seed(1)
    lin = BlockFHTLinear(96, 40, latent_dim=1000, layers=2, seed=5, weight_scale=0.7, **opts).cuda()
    with torch.no_grad():
        if lin.bias is not None:
            lin.bias.normal_()
        for gain in (lin.output_gain, lin.input_gain):
            if gain is not None:
                gain.uniform_(0.5, 1.5)
        x = torch.randn(3, 7, 96, device="cuda")
        got = lin.forward_fused(x)
        want = torch.nn.functional.linear(x.double(), lin.weight.double(),
                                          None if lin.bias is None else lin.bias.double())
    assert got.shape == (3, 7, 40)
    assert O.rel_l2(got.double().cpu().numpy(), want.cpu().numpy()) < 1e-5
