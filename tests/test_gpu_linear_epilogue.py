"""GPU parity of the fused linear's epilogue (``lwl_bfht_linear_forward_ex``): the modulation
term, the residual base and the bias of ``BlockFHTLinear.forward_fused`` (reference
latent_weight_lab/block_fht.py:493-500) added in the fused kernels' stores.

1. Every term alone and all together, in both fused domains (bf16 block 2^15 on the matrix
   cores, with rows that straddle blocks, untiled and tiled batches; the reference's own
   float32 / float16 / bfloat16 domain), against ``base + scale * x @ W^T + c * x.sum(-1) +
   bias`` in float64 with W from the C oracle.  Each term is drawn about as large as the
   product, so a missing, doubled or misplaced term fails the bar (bf16 1e-2, f16 2e-3,
   f32 1e-5 relative L2).
2. Float32: the epilogue output minus the plain output equals the terms to float32 rounding,
   element by element (a sharp check of the arithmetic and the indexing).
3. Grouped calls with per-job epilogues equal their single calls bit for bit.
4. ``forward_fused`` of modules with bias, modulation and residual base, under ``no_grad`` (one
   fused launch) and recording gradients (the reference's sequence of ops), against the
   float64 truth.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import BlockFHTLinear, forward_fused_grouped, ops
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1e-2}

CASES = [
    # (dtype, tokens, in, out, latent, layers, seed, scale)
    (torch.bfloat16, 64, 768, 3072, 32768, 3, 3, 1.0),     # matrix cores, untiled, straddling rows
    (torch.bfloat16, 4096, 768, 3072, 32768, 3, 3, 1.0),   # tiled x, 64-row tiles (NT 4)
    (torch.bfloat16, 320, 704, 64, 32768, 3, 37, 1.0),     # two blocks, 6 row tiles: base and bias loads branched
    (torch.bfloat16, 300, 1000, 77, 30000, 2, 8, 1.0),     # two blocks, 5 row tiles, rows straddle blocks
    (torch.bfloat16, 300, 3072, 768, 32768, 3, 4, 0.5),    # tiled, 3072 -> 768
    (torch.bfloat16, 3100, 3072, 700, 32768, 3, 4, 0.5),   # three-block tiles, last tile 28 rows
    (torch.bfloat16, 17, 528, 200, 30000, 2, 5, 2.0),      # ragged tokens, one partial block
    (torch.float32, 300, 1024, 4096, 16384, 2, 123, 0.5),  # reference domain
    (torch.float16, 37, 64, 200, 4096, 3, -3, 1.0),
    (torch.bfloat16, 37, 64, 200, 4096, 3, -3, 1.0),
    (torch.float16, 256, 64, 200, 4096, 3, -3, 1.0),      # reference domain on the matrix cores, tiled x
    (torch.bfloat16, 100, 256, 1000, 2000, 2, 5, 1.0),    # reference domain on the matrix cores, row-major x
]

TERMS = [("bias",), ("base",), ("row_sum",), ("bias", "base", "row_sum")]


def weight64(latent: torch.Tensor, in_f: int, out_f: int, layers: int, seed: int) -> np.ndarray:
    w = c_oracle.forward(latent.double().cpu().numpy(), in_f * out_f, layers, seed, 0, in_f * out_f)
    return w.reshape(out_f, in_f)


def make_terms(gen, dtype, tokens, out_f, in_f, sigma, which):
    """Epilogue tensors about as large as the product (standard deviation sigma each)."""
    kw = {}
    if "bias" in which:
        kw["bias"] = (sigma * torch.randn(out_f, generator=gen)).to(dtype).cuda()
    if "base" in which:
        kw["base"] = (sigma * torch.randn(tokens, out_f, generator=gen)).to(dtype).cuda()
    if "row_sum" in which:
        # c * x.sum(-1) ~ sigma: x.sum has standard deviation sqrt(in)
        kw["row_sum_coef"] = torch.tensor([0.7 * sigma / np.sqrt(in_f)], dtype=torch.float32).cuda()
        kw["row_sum_scale"] = 1.5
    return kw


def truth(x, w64, scale, kw):
    xd = x.double().cpu().numpy()
    out = scale * (xd @ w64.T)
    if "row_sum_coef" in kw:
        c = float(kw["row_sum_coef"].item()) * kw["row_sum_scale"]
        out = out + c * xd.sum(axis=1, keepdims=True)
    if "base" in kw:
        out = out + kw["base"].double().cpu().numpy()
    if "bias" in kw:
        out = out + kw["bias"].double().cpu().numpy()[None, :]
    return out


@pytest.mark.parametrize("dtype,tokens,in_f,out_f,n,layers,seed,scale", CASES)
def test_epilogue_terms_match_oracle(dtype, tokens, in_f, out_f, n, layers, seed, scale):
    gen = torch.Generator().manual_seed(tokens + in_f + out_f)
    latent = torch.randn(n, generator=gen).to(dtype)
    x = torch.randn(tokens, in_f, generator=gen).to(dtype)
    assert ops.linear_supported(in_f, out_f, latent.cuda(), x.cuda())
    w64 = weight64(latent, in_f, out_f, layers, seed)
    sigma = float(np.std(scale * (x[:8].double().numpy() @ w64.T)))
    xd, ld = x.cuda(), latent.cuda()
    for which in TERMS:
        kw = make_terms(gen, dtype, tokens, out_f, in_f, sigma, which)
        got = ops.linear_forward(xd, ld, out_f, layers, seed, scale, **kw)
        err = O.rel_l2(got.double().cpu().numpy(), truth(x, w64, scale, kw))
        assert err < TOL[dtype], (which, dtype, tokens, in_f, out_f, err)


def test_epilogue_float32_elementwise():
    """out_ex - out_plain = the terms, to float32 rounding, element by element."""
    gen = torch.Generator().manual_seed(11)
    tokens, in_f, out_f, n, layers, seed, scale = 300, 1024, 4096, 16384, 2, 123, 0.5
    latent = torch.randn(n, generator=gen).cuda()
    x = torch.randn(tokens, in_f, generator=gen).cuda()
    plain = ops.linear_forward(x, latent, out_f, layers, seed, scale).double()
    kw = make_terms(gen, torch.float32, tokens, out_f, in_f, float(plain.std()), TERMS[-1])
    got = ops.linear_forward(x, latent, out_f, layers, seed, scale, **kw).double()
    c = float(kw["row_sum_coef"].item()) * kw["row_sum_scale"]
    row = c * x.double().sum(dim=1, keepdim=True)
    base, bias = kw["base"].double(), kw["bias"].double()[None, :]
    terms = row + base + bias
    # each of the three adds rounds once (at most the running magnitude times 2^-24); the
    # row sum is a float32 tree of depth ~10 over `in` values, then two products
    mag = plain.abs() + row.abs() + base.abs() + bias.abs()
    bound = 2.0 ** -21 * mag + 2.0 ** -18 * abs(c) * x.double().abs().sum(1, keepdim=True)
    assert bool(((got - plain - terms).abs() <= bound).all())


def test_epilogue_none_is_plain():
    gen = torch.Generator().manual_seed(12)
    latent = torch.randn(32768, generator=gen).to(torch.bfloat16).cuda()
    x = torch.randn(40, 768, generator=gen).to(torch.bfloat16).cuda()
    a = ops.linear_forward(x, latent, 3072, 3, 3, 1.0)
    b = ops.linear_forward(x, latent, 3072, 3, 3, 1.0, bias=None, base=None, row_sum_coef=None)
    assert torch.equal(a, b)


def test_grouped_epilogues_equal_single_calls():
    """Bias-only jobs run in the grouped kernels, base / row-sum jobs as single launches
    inside the call; every output equals its single call bit for bit."""
    gen = torch.Generator().manual_seed(13)
    lat_a = torch.randn(32768, generator=gen).to(torch.bfloat16).cuda()
    lat_b = torch.randn(30000, generator=gen).to(torch.bfloat16).cuda()
    cases = [  # (tokens, in, out, latent, layers, seed, scale, terms)
        (3, 768, 2304, lat_a, 3, 1, 1.0, ("bias",)),
        (17, 768, 768, lat_a, 2, 2, 0.5, ()),
        (1, 3072, 768, lat_b, 3, 3, 1.0, ("bias",)),
        (40, 528, 200, lat_b, 1, 4, 2.0, ("base",)),
        (64, 2048, 90, lat_b, 2, 7, 0.25, ("bias", "base", "row_sum")),
        (300, 1024, 300, lat_a, 3, 6, 1.0, ("bias",)),   # tiled x: single launch
    ]
    specs = []
    for t, i, o, lat, L, sd, sc, which in cases:
        x = torch.randn(t, i, generator=gen).to(torch.bfloat16).cuda()
        kw = make_terms(gen, torch.bfloat16, t, o, i, 10.0, which)
        specs.append((x, lat, o, L, sd, sc, kw))
    grouped = ops.linear_forward_grouped(specs)
    for sp, got in zip(specs, grouped):
        assert torch.equal(got, ops.linear_forward(*sp[:6], **sp[6])), sp[1:6]


def module(in_f, out_f, n, dtype, seed, **opts):
    torch.manual_seed(seed)
    m = BlockFHTLinear(in_f, out_f, bias=True, latent_dim=n, layers=3, seed=seed, **opts)
    with torch.no_grad():
        m.generator.latent.normal_()
        m.bias.normal_(0.0, 10.0)
    return m.cuda().to(dtype)


def module_truth(m, x):
    """float64 forward_fused of the reference (block_fht.py:482-501) from the oracle's weight."""
    g = m.generator
    w64 = weight64(g.latent.detach(), m.in_features, m.out_features, g.layers, g.seed) * m.weight_scale
    xd = x.reshape(-1, m.in_features).double().cpu().numpy()
    out = xd @ w64.T
    if m.modulation_alpha != 0.0:
        mod = (m.modulation_alpha * m._modulation_offset()).to(x.dtype).double().item()
        out = out + mod * xd.sum(axis=1, keepdims=True)
    if m.residual_base_weight is not None:
        out = xd @ m.residual_base_weight.double().cpu().numpy().T + m.residual_base_scale * out
    return out + m.bias.detach().double().cpu().numpy()[None, :]


@pytest.mark.parametrize("dtype,in_f,out_f,n", [(torch.bfloat16, 768, 3072, 32768), (torch.bfloat16, 3072, 768, 32768),
                                                 (torch.float32, 1024, 4096, 16384)])
@pytest.mark.parametrize("tokens", [1, 64, 2048])
def test_forward_fused_module_epilogue(dtype, in_f, out_f, n, tokens):
    m = module(in_f, out_f, n, dtype, 21, modulation_alpha=3e-5, residual_base_scale=0.5, residual_base_std=1.0)
    x = torch.randn(2, tokens // 2 if tokens > 1 else 1, in_f, device="cuda").to(dtype)
    want = module_truth(m, x)
    with torch.no_grad():
        fused = m.forward_fused(x)
    assert fused.shape == (*x.shape[:-1], out_f) and fused.dtype == dtype
    err = O.rel_l2(fused.reshape(-1, out_f).double().cpu().numpy(), want)
    assert err < TOL[dtype], ("no_grad", err)
    # recording gradients: the reference's sequence of ops after the fused (or generated) linear
    seq = m.forward_fused(x.requires_grad_(True))
    err2 = O.rel_l2(seq.detach().reshape(-1, out_f).double().cpu().numpy(), want)
    assert err2 < TOL[dtype], ("grad", err2)


def test_forward_fused_grouped_with_epilogues():
    mods = [module(768, 2304, 32768, torch.bfloat16, 1),
            module(768, 768, 32768, torch.bfloat16, 2, modulation_alpha=3e-5),
            module(3072, 768, 32768, torch.bfloat16, 3, residual_base_scale=0.5, residual_base_std=1.0),
            module(768, 3072, 32768, torch.bfloat16, 4)]
    xs = [torch.randn(5, m.in_features, device="cuda").to(torch.bfloat16) for m in mods]
    with torch.no_grad():
        got = forward_fused_grouped(mods, xs, weight_scale=0.5)
        want = [m.forward_fused(x, weight_scale=0.5) for m, x in zip(mods, xs)]
    for g_, w_ in zip(got, want):
        assert torch.equal(g_, w_)
