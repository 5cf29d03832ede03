"""GPU parity of the fused linear in the reference extension's own domain, and of the
fused route's gradients.

1. ``lwl_bfht_linear_forward`` for float32 / float16 / bfloat16 latents of block <= 2^14 with
   ``block_size % in_features == 0`` (the reference gate latent_weight_lab/block_fht.py:263-273,
   kernel csrc/block_fht_ext_cuda.cu:225-329): the weight is generated in float32 into LDS and
   contracted there.  Checked against ``x @ (scale * W)^T`` in float64 with W from the C oracle
   (same dtype-rounded latent): float32 1e-5 relative L2, float16 2e-3 and bfloat16 1e-2 (one
   output rounding; the BASELINE bar for 16-bit types is 1e-2).  Called through the ctypes shim
   that INTEGRATION.md gives for the reference (Option B), under the reference's unchanged gate,
   at the reference tests' shapes (tests/test_block_fht_cuda.py:43-98) and its profiling case
   (scripts/profile_fused_once.py:10-13: 1024 -> 4096, float16, latent 16384, scale 0.5).
2. The reference module tests of ``forward_fused`` (tests/test_block_fht_cuda.py:43-98) with
   their own tolerances.
3. Gradients through the fused route at the north-star shapes (bf16, block 2^15, 768 -> 3072
   and 3072 -> 768, 4096 tokens): latent, input and bias gradients against float32 / float64
   products with the oracle's weight and the oracle's adjoint, 1e-2 relative L2 — the reference
   gives these gradients through its differentiable fallback (block_fht.py:282-288).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import BlockFHTLinear, block_fht_linear_forward
from latent_weight_lab_amd import _native as N
from latent_weight_lab_amd import ops
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1e-2}


@pytest.fixture(scope="module")
def ext():
    from ext_shim import _LwlExt

    N.lib()  # torch's HIP runtime first, then the library (same SONAME)
    return _LwlExt(str(N.library_path()))


def reference_gate(latent: torch.Tensor, in_features: int) -> bool:
    """block_fht.py:263-273: the reference calls ext.linear_forward only here."""
    block = ops.next_power_of_two(latent.numel())
    return block <= 16384 and block % in_features == 0


def oracle_out(x: torch.Tensor, latent: torch.Tensor, out_f: int, layers: int, seed: int, scale: float):
    in_f = x.shape[-1]
    w = c_oracle.forward(latent.double().cpu().numpy(), in_f * out_f, layers, seed, 0, in_f * out_f)
    return (x.reshape(-1, in_f).double().cpu().numpy() @ w.reshape(out_f, in_f).T) * scale


CASES = [
    # (tokens, in, out, latent, layers, seed, scale)
    (5, 8, 6, 32, 2, 8, 0.125),        # reference test shapes (block 32 = 4 rows of 8)
    (11, 8, 6, 32, 2, 9, 0.5),
    (12, 8, 6, 32, 1, 7, 1.0),         # batched 3 x 4 tokens
    (1, 1024, 4096, 16384, 2, 123, 0.5),  # reference profiling case (scripts/profile_fused_once.py)
    (300, 1024, 4096, 16384, 2, 123, 0.5),  # the same with a batch: token splits
    (37, 64, 200, 4096, 3, -3, 1.0),   # 64 rows per block, partial last block (200 rows); matrix cores
    (13, 64, 200, 4096, 3, -3, 1.0),   # the same on VALU: a single-token last quad, teams' second rows past the tile
    (12, 2048, 40, 16384, 3, 7, 1.0),  # x of a quad staged in two rounds of loads, three quads
    (130, 16384, 5, 16384, 1, 11, 2.0),  # one row per block
    (9, 1, 7, 1, 3, 4, 1.0),           # block 2^0
    (70, 2, 300, 3, 2, 5, 1.0),        # block 2^2: 256 blocks per workgroup
    (1000, 32, 2000, 500, 3, 6, 0.75),  # block 2^9 (16 rows of 32), 16 blocks per workgroup
    (3, 4096, 3, 8000, 2, 12, 1.0),    # block 2^13, out smaller than one block
    # from 16 tokens the contraction runs on the matrix cores (bfht_linear_small_mm) where
    # in_features is a multiple of 32 (16 for float32) with >= 16 rows per workgroup tile
    (256, 64, 200, 4096, 3, -3, 1.0),   # block 2^12: 200 of 512 table rows, 13 row tiles
    (100, 256, 1000, 2000, 2, 5, 1.0),  # block 2^11, ragged token tiles
    (64, 2048, 40, 16384, 3, 7, 1.0),   # 16 rows per 16-bit tile; float32 (8 rows) stays on VALU
    (2048, 128, 512, 1024, 2, 9, 0.5),  # block 2^10, token splits
    (80, 16, 64, 64, 1, 10, 1.0),       # in 16: float32 on the matrix cores, 16-bit on VALU
    # block 2^5, the matrix-core kernel's smallest: 256 blocks per generator call, 4 calls per tile
    (64, 32, 48, 32, 2, 3, 1.0),        # 16-bit and float32 on the matrix cores (48 of 1024 table rows)
    (80, 16, 40, 32, 1, 4, 1.0),        # float32 on the matrix cores, 16-bit on VALU
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tokens,in_f,out_f,n,layers,seed,scale", CASES)
def test_reference_domain_through_shim(ext, dtype, tokens, in_f, out_f, n, layers, seed, scale):
    g = torch.Generator().manual_seed(tokens * 7 + in_f)
    latent = torch.randn(n, generator=g).to(dtype)
    x = torch.randn(tokens, in_f, generator=g).to(dtype)
    xd, ld = x.cuda(), latent.cuda()
    assert reference_gate(ld, in_f), "the reference would call ext.linear_forward here"
    got = ext.linear_forward(xd, ld, out_f, layers, seed, scale)
    torch.cuda.synchronize()
    assert got.shape == (tokens, out_f) and got.dtype == dtype
    want = oracle_out(x, latent, out_f, layers, seed, scale)
    assert O.rel_l2(got.double().cpu().numpy(), want) < TOL[dtype]
    # the package's fused route is the same kernel
    pkg = block_fht_linear_forward(xd, ld, out_f, layers, seed, weight_scale=scale, fused=True)
    assert torch.equal(pkg, got)


def test_shim_forward_backward_at_reference_test_shapes(ext):
    # reference tests/test_block_fht_cuda.py:10-31 through the shim (fp32, layers 1, seed 123)
    for n, size, start, stop in ((4096, 8192, 17, 4099), (20000, 65536, 111, 4096)):
        torch.manual_seed(0)
        lat = torch.randn(n, dtype=torch.float32)
        y = ext.forward(lat.cuda(), size, 1, 123, start, stop)[0]
        want = c_oracle.forward(lat.double().numpy(), size, 1, 123, start, stop)
        assert O.rel_l2(y.double().cpu().numpy(), want) < 1e-5
        g = ext.backward((2 * y).contiguous(), n, size, 1, 123, start, stop)
        gwant = c_oracle.backward(2 * want, n, size, 1, 123, start, stop)
        assert O.rel_l2(g.double().cpu().numpy(), gwant) < 1e-5


def test_shim_raises_outside_the_kernels(ext):
    # a shape the reference gate sends to the extension is never refused; outside every kernel's
    # domain the C ABI reports unsupported with a message
    lat = torch.randn(32768, device="cuda")
    x = torch.randn(4, 768, device="cuda")
    with pytest.raises(RuntimeError, match="fused linear forward takes"):
        ext.linear_forward(x, lat, 64, 2, 1, 1.0)


# ---------------------------------------------------------------- reference module tests

def test_cuda_fused_linear_forward_matches_materialized_weight():
    torch.manual_seed(123)
    layer = BlockFHTLinear(7, 5, bias=True, latent_dim=32, layers=2, seed=99).cuda()
    x = torch.randn(11, 7, device="cuda")
    fused = layer.forward_fused(x)
    materialized = layer(x)
    torch.cuda.synchronize()
    assert torch.allclose(fused, materialized, atol=2e-5, rtol=2e-5)


def test_cuda_fused_linear_forward_supports_batched_input():
    torch.manual_seed(321)
    layer = BlockFHTLinear(8, 6, bias=False, latent_dim=32, layers=1, seed=7).cuda()
    x = torch.randn(3, 4, 8, device="cuda")
    assert ops.linear_supported(8, 6, layer.generator.latent, x)
    fused = layer.forward_fused(x)
    materialized = layer(x)
    torch.cuda.synchronize()
    assert fused.shape == (3, 4, 6)
    assert torch.allclose(fused, materialized, atol=2e-5, rtol=2e-5)


def test_cuda_fused_linear_forward_supports_weight_scale():
    torch.manual_seed(456)
    layer = BlockFHTLinear(8, 6, bias=False, latent_dim=32, layers=2, seed=8).cuda()
    x = torch.randn(5, 8, device="cuda")
    scale = 0.125
    fused = layer.forward_fused(x, weight_scale=scale)
    materialized = torch.nn.functional.linear(x, layer.weight * scale)
    torch.cuda.synchronize()
    assert torch.allclose(fused, materialized, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("dtype,atol", [(torch.float16, 2e-3), (torch.bfloat16, 2e-2)])
def test_cuda_fused_linear_forward_supports_16bit(dtype, atol):
    torch.manual_seed(789)
    layer = BlockFHTLinear(8, 6, bias=False, latent_dim=32, layers=2, seed=9).cuda().to(dtype)
    x = torch.randn(5, 8, device="cuda", dtype=dtype)
    scale = 0.5
    fused = layer.forward_fused(x, weight_scale=scale)
    materialized = torch.nn.functional.linear(x.float(), layer.weight.float() * scale).to(dtype)
    torch.cuda.synchronize()
    assert fused.dtype == dtype
    assert torch.allclose(fused, materialized, atol=atol, rtol=atol)


# ---------------------------------------------------------------- gradients through the fused route

@pytest.mark.parametrize("in_f,out_f", [(768, 3072), (3072, 768)])
def test_fused_route_gradients_north_star(in_f, out_f):
    tokens, layers, seed, scale = 4096, 3, 3, 0.5
    g = torch.Generator().manual_seed(in_f)
    lat = torch.randn(32768, generator=g).to(torch.bfloat16)
    lin = BlockFHTLinear(in_f, out_f, bias=True, latent_dim=32768, layers=layers, seed=seed,
                         weight_scale=scale).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.generator.latent.copy_(lat.cuda())
        lin.bias.copy_(torch.randn(out_f, generator=g).to(torch.bfloat16).cuda())
    x = torch.randn(tokens, in_f, generator=g).to(torch.bfloat16).cuda().requires_grad_(True)
    assert ops.linear_supported(in_f, out_f, lin.generator.latent, x), "the fused kernel takes this shape"
    y = lin.forward_fused(x)
    assert y.requires_grad, "the fused route records an autograd graph"
    r = torch.randn(tokens, out_f, generator=g).to(torch.bfloat16).cuda()
    y.backward(r)
    torch.cuda.synchronize()

    size = in_f * out_f
    w = c_oracle.forward(lat.double().numpy(), size, layers, seed, 0, size).reshape(out_f, in_f)
    wd = torch.from_numpy(w).float().cuda() * scale
    rf, xf = r.float(), x.detach().float()
    want_y = xf @ wd.t() + lin.bias.detach().float()
    assert O.rel_l2(y.detach().double().cpu().numpy(), want_y.double().cpu().numpy()) < 1e-2
    want_gx = rf @ wd
    assert O.rel_l2(x.grad.double().cpu().numpy(), want_gx.double().cpu().numpy()) < 1e-2
    gw = (rf.t() @ xf).double().cpu().numpy().reshape(-1)
    want_gl = scale * c_oracle.backward(gw, 32768, size, layers, seed, 0, size)
    assert O.rel_l2(lin.generator.latent.grad.double().cpu().numpy(), want_gl) < 1e-2
    want_gb = rf.sum(dim=0)
    assert O.rel_l2(lin.bias.grad.double().cpu().numpy(), want_gb.double().cpu().numpy()) < 1e-2


def test_fused_route_without_grad_records_nothing():
    lat = torch.randn(32768, device="cuda").to(torch.bfloat16)
    x = torch.randn(16, 768, device="cuda").to(torch.bfloat16)
    y = block_fht_linear_forward(x, lat, 3072, 3, 1)
    assert y.grad_fn is None
    lat.requires_grad_(True)
    with torch.no_grad():
        assert block_fht_linear_forward(x, lat, 3072, 3, 1).grad_fn is None
    y = block_fht_linear_forward(x, lat, 3072, 3, 1)
    assert y.grad_fn is not None
    y.float().sum().backward()
    assert lat.grad is not None and torch.isfinite(lat.grad.float()).all()


def test_small_domain_gradients_match_generated_route():
    # fp32, block 2^12, in | block: the fused route's gradients equal the generate + F.linear
    # route's (both differentiable, reference block_fht.py:282-288) within the float32 bar
    g = torch.Generator().manual_seed(3)
    lat = torch.randn(4000, generator=g).cuda()
    x = torch.randn(50, 256, generator=g).cuda()
    grads = []
    for fused in (True, False):
        la = lat.clone().requires_grad_(True)
        xa = x.clone().requires_grad_(True)
        y = block_fht_linear_forward(xa, la, 100, 2, 9, weight_scale=0.5, fused=fused)
        y.square().sum().backward()
        grads.append((y.detach(), la.grad, xa.grad))
    for a, b in zip(*grads):
        assert O.rel_l2(a.double().cpu().numpy(), b.double().cpu().numpy()) < 1e-5
