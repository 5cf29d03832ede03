"""GPU parity of the grouped weight cache: prepare / flush of many BlockFHTLinear
modules in a few launches (reference latent_weight_lab/block_fht.py:503-569, whose
loops call ext.forward / ext.backward once per module).

The grouped kernels run every block with the code of the per-module launch, and
fold in torch's ``* weight_scale``, ``.to(dtype)`` and ``latent.grad.add_`` with
the same roundings, so the bar is bit-identity (``torch.equal``) with the
per-module path; one job per dtype is also checked against the C oracle
(float32 1e-5, bf16 / fp16 1e-2 relative L2, as the per-module tests).
"""
from __future__ import annotations

import copy

import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import (BlockFHTLinear, block_fht_grad_latent, flush_block_fht_weight_cache,
                                   prepare_block_fht_weight_cache)
from latent_weight_lab_amd import ops
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

F32, F16, BF16 = torch.float32, torch.float16, torch.bfloat16

# (latent size, size, layers, seed, weight_scale, latent dtype, weight dtype)
JOBS = [
    (23593, 768 * 3072, 2, 1000, 1.0, F32, BF16),     # GPT-2 MLP at latent ratio 0.01: block 2^15, fp32 latent
    (5898, 768 * 768, 2, 1001, 0.25, F32, BF16),      # block 2^13, one block per workgroup
    (17694, 768 * 2304, 3, 1002, 1.0, F32, F32),      # fp32 cache
    (32768, 1024 * 1024, 3, 7, 0.5, BF16, BF16),      # bf16 block 2^15: matrix cores, scaled
    (20000, 300 * 1000, 2, 8, 1.0, BF16, BF16),       # matrix cores, padded latent, partial last block
    (3000, 64 * 500, 1, 9, 2.0, F16, F32),            # fp16 latent, block 2^12 (2 blocks per workgroup)
    (10, 7 * 33, 3, -4, 1.0, F32, F16),               # block 2^4 (256 blocks per workgroup), partial
    (1, 5, 2, 3, 1.5, F32, F32),                      # one-element latent, block 2^0
    (4096, 4096, 3, 11, 1.0, BF16, F32),              # bf16 latent, block 2^12, fp32 cache
    (32768, 300 * 1000, 3, 12, 0.75, BF16, BF16),     # matrix cores, odd L: whole blocks stored from
                                                      # registers, the partial last one staged; scaled
    (30000, 512 * 700, 1, 13, 1.0, BF16, BF16),       # matrix cores, one layer, partial last block
]


def make_latent(n, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * 0.02).to(dtype).cuda()


def per_module_weight(latent, size, layers, seed, ws, wdtype):
    return (ops.forward(latent, size, layers, seed, 0, size) * ws).to(wdtype)


def test_materialize_matches_per_module_bitwise():
    latents = [make_latent(n, ld, i) for i, (n, _, _, _, _, ld, _) in enumerate(JOBS)]
    specs = [(lat, size, layers, seed, ws, wd) for lat, (_, size, layers, seed, ws, _, wd) in zip(latents, JOBS)]
    got = ops.materialize_weights(specs)
    torch.cuda.synchronize()
    for spec, w in zip(specs, got):
        want = per_module_weight(*spec)
        assert w.dtype == want.dtype and w.shape == want.shape
        assert torch.equal(w, want), spec[1:]


@pytest.mark.parametrize("ld,tol", [(F32, 1e-5), (BF16, 1e-2), (F16, 1e-2)])
def test_materialize_matches_oracle(ld, tol):
    n, size, layers, seed, ws = 30000, 200 * 700, 3, 17, 0.5
    lat = make_latent(n, ld, 5)
    (w,) = ops.materialize_weights([(lat, size, layers, seed, ws, ld)])
    want = ws * c_oracle.forward(lat.double().cpu().numpy(), size, layers, seed, 0, size)
    assert O.rel_l2(w.double().cpu().numpy(), want) < tol


def test_flush_matches_per_module_bitwise():
    latents = [make_latent(n, ld, 50 + i) for i, (n, _, _, _, _, ld, _) in enumerate(JOBS)]
    grads = []
    for i, (n, size, *_rest, wd) in enumerate(JOBS):
        g = torch.Generator().manual_seed(100 + i)
        grads.append(torch.randn(size, generator=g).to(wd).cuda())
    # half the jobs add into an existing gradient
    intos = [None if i % 2 else (torch.randn(lat.numel()) * 0.1).to(lat.dtype).cuda()
             for i, lat in enumerate(latents)]
    before = [None if t is None else t.clone() for t in intos]
    specs = [(lat, gw, size, layers, seed, ws, into)
             for lat, gw, into, (_, size, layers, seed, ws, _, _) in zip(latents, grads, intos, JOBS)]
    got = ops.flush_weight_grads(specs)
    torch.cuda.synchronize()
    for i, ((lat, gw, size, layers, seed, ws, into), r) in enumerate(zip(specs, got)):
        want = ws * block_fht_grad_latent(lat, gw.to(lat.dtype), size, layers, seed)
        if before[i] is not None:
            want = before[i].add_(want)
            assert r.data_ptr() == into.data_ptr()
        assert r.dtype == lat.dtype
        assert torch.equal(r, want), JOBS[i]


@pytest.mark.parametrize("ld,tol", [(F32, 1e-5), (BF16, 1e-2)])
def test_flush_matches_oracle(ld, tol):
    n, size, layers, seed, ws = 30000, 200 * 700, 2, 23, 2.0
    lat = make_latent(n, ld, 6)
    gw = torch.randn(size, generator=torch.Generator().manual_seed(7)).to(ld).cuda()
    (r,) = ops.flush_weight_grads([(lat, gw, size, layers, seed, ws, None)])
    want = ws * c_oracle.backward(gw.double().cpu().numpy(), n, size, layers, seed, 0, size)
    assert O.rel_l2(r.double().cpu().numpy(), want) < tol


def test_more_jobs_than_one_table():
    # 40 generators: the planner splits them over two launch tables
    specs, lats = [], []
    for i in range(40):
        n = 100 + 37 * i
        lat = make_latent(n, F32, 200 + i)
        lats.append(lat)
        specs.append((lat, 3 * n + i, 1 + i % 3, i, 1.0, F32))
    got = ops.materialize_weights(specs)
    grads = [torch.randn_like(w) for w in got]
    flushed = ops.flush_weight_grads([(lat, g, s[1], s[2], s[3], 1.0, None)
                                      for lat, g, s in zip(lats, grads, specs)])
    torch.cuda.synchronize()
    for s, w, g, r in zip(specs, got, grads, flushed):
        assert torch.equal(w, per_module_weight(*s))
        assert torch.equal(r, block_fht_grad_latent(s[0], g, s[1], s[2], s[3]))


class Net(torch.nn.Module):
    """Modules of every cache kind: plain fp32 latents (grouped, cast to bf16),
    gains and modulation (grouped with torch epilogues), a residual base (never
    cached), and a latent above 2^15 (per-module tile path)."""

    def __init__(self):
        super().__init__()
        self.qkv = BlockFHTLinear(768, 2304, latent_ratio=0.01, layers=2, seed=1, weight_scale=0.5)
        self.fc = BlockFHTLinear(768, 3072, latent_ratio=0.01, layers=2, seed=2)
        self.proj = BlockFHTLinear(3072, 768, latent_ratio=0.01, layers=2, seed=3, output_gain=True,
                                   input_gain=True)
        self.mod = BlockFHTLinear(256, 512, latent_ratio=0.05, layers=3, seed=4, modulation_alpha=0.1)
        self.res = BlockFHTLinear(256, 256, latent_ratio=0.05, layers=1, seed=5, residual_base_scale=0.5)
        self.big = BlockFHTLinear(1024, 1024, latent_dim=50000, layers=2, seed=6)

    def forward(self, x, y, z):
        h = self.qkv(x).float().sum() + self.fc(x).float().sum() * 0.5
        h = h + self.proj(y).float().pow(2).sum() * 1e-3
        h = h + self.mod(z).float().sum() + self.res(z).float().sum() + self.big(
            torch.cat([z, z, z, z], dim=-1)).float().sum()
        return h


def per_module_prepare(model, dtype):
    for m in model.modules():
        if isinstance(m, BlockFHTLinear):
            m.materialize_weight_cache(dtype=dtype)


def per_module_flush(model):
    for m in model.modules():
        if isinstance(m, BlockFHTLinear):
            m.flush_weight_cache_to_latent_grad()


@pytest.mark.parametrize("cache_dtype", [BF16, None])
def test_model_prepare_flush_matches_per_module(cache_dtype):
    torch.manual_seed(0)
    a = Net().cuda()
    with torch.no_grad():
        for m in a.modules():
            if isinstance(m, BlockFHTLinear) and m.output_gain is not None:
                m.output_gain.uniform_(0.5, 1.5)
                m.input_gain.uniform_(0.5, 1.5)
    b = copy.deepcopy(a)
    x = torch.randn(8, 768, device="cuda")
    y = torch.randn(8, 3072, device="cuda")
    z = torch.randn(8, 256, device="cuda")
    # a: grouped helpers; b: the per-module loop; two microbatches each, the
    # second flush adding into the gradients of the first
    for step in range(2):
        prepare_block_fht_weight_cache(a, dtype=cache_dtype)
        per_module_prepare(b, cache_dtype)
        for (na, ma), (nb, mb) in zip(a.named_modules(), b.named_modules()):
            if isinstance(ma, BlockFHTLinear):
                assert (ma._cached_weight is None) == (mb._cached_weight is None), na
                if ma._cached_weight is not None:
                    assert torch.equal(ma._cached_weight, mb._cached_weight), na
        cast = (lambda t: t.to(cache_dtype)) if cache_dtype is not None else (lambda t: t)
        a(cast(x), cast(y), cast(z)).backward()
        b(cast(x), cast(y), cast(z)).backward()
        flush_block_fht_weight_cache(a)
        per_module_flush(b)
        for (na, pa), (nb, pb) in zip(a.named_parameters(), b.named_parameters()):
            assert (pa.grad is None) == (pb.grad is None), na
            if pa.grad is not None:
                assert torch.equal(pa.grad, pb.grad), (step, na)
    for m in a.modules():
        if isinstance(m, BlockFHTLinear):
            assert m._cached_weight is None


def test_flush_weight_gradients_off_the_16_byte_grid_bitwise():
    """bf16 weight gradients of block-2^15 jobs that are views at 2- and 6-byte offsets
    (and one aligned) run on the matrix cores in both paths, which read them as aligned
    16-byte slots: the grouped flush stays bit-identical to the per-module backward."""
    sizes = [1024 * 1024, 300 * 1000 + 13, 768 * 3072]
    offsets = [1, 3, 0]
    base = torch.randn(sum(sizes) + 256, generator=torch.Generator().manual_seed(41)).to(BF16).cuda()
    specs, at = [], 0  # `at` stays a multiple of 8 elements (16 bytes) from the 256-byte aligned base
    for i, (size, off) in enumerate(zip(sizes, offsets)):
        gw = base[at + off: at + off + size]
        assert gw.data_ptr() % 16 == 2 * off
        at = (at + off + size + 15) // 8 * 8
        lat = make_latent(32768 if i != 1 else 20000, BF16, 60 + i)
        specs.append((lat, gw, size, 3, 70 + i, 0.5 if i else 1.0, None))
    got = ops.flush_weight_grads(specs)
    torch.cuda.synchronize()
    for (lat, gw, size, layers, seed, ws, _), r in zip(specs, got):
        want = ws * block_fht_grad_latent(lat, gw, size, layers, seed)
        assert torch.equal(r, want), (size, gw.data_ptr() % 16)


# ---------------------------------------------------------------- reference module tests, on the GPU

def _rel(a, b):
    return O.rel_l2(a.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())


def _check_close(got, want, dtype):
    # reference bar: allclose(atol=1e-6) on float32 CPU tensors; bf16 runs at the 1e-2 rel-L2 bar
    if dtype == F32:
        assert torch.allclose(got, want, atol=1e-6, rtol=1e-5), _rel(got, want)
    else:
        assert _rel(got, want) < 1e-2


def _gain_pair(dtype, shape_kw):
    kw = dict(bias=True, layers=2, seed=13, output_gain=True, input_gain=True, modulation_alpha=1e-3,
              modulation_centered=True, **shape_kw)
    dynamic = BlockFHTLinear(**kw).cuda()
    with torch.no_grad():
        dynamic.output_gain.copy_(torch.linspace(0.7, 1.3, dynamic.out_features))
        dynamic.input_gain.copy_(torch.linspace(0.6, 1.4, dynamic.in_features))
    dynamic = dynamic.to(dtype)
    cached = BlockFHTLinear(**kw).cuda().to(dtype)
    cached.load_state_dict(dynamic.state_dict())
    return dynamic, cached


@pytest.mark.parametrize("dtype,shape_kw", [
    (F32, dict(in_features=5, out_features=3, latent_dim=8)),           # the reference's shape
    (F32, dict(in_features=768, out_features=768, latent_dim=5898)),    # GPT-2 proj at latent ratio 0.01
    (BF16, dict(in_features=768, out_features=3072, latent_dim=32768)),  # matrix-core generator
])
def test_cached_grad_matches_dynamic_with_channel_gains(dtype, shape_kw):
    """Reference tests/test_block_fht.py:100-143 (and :78-97 without gains): the prepare ->
    forward/backward -> flush path gives the latent, bias and both gains the gradients of the
    dynamic (uncached) module."""
    torch.manual_seed(321)
    dynamic, cached = _gain_pair(dtype, shape_kw)
    x = torch.randn(4, dynamic.in_features, device="cuda").to(dtype)

    dynamic_loss = dynamic(x).float().square().mean()
    dynamic_loss.backward()

    prepare_block_fht_weight_cache(cached)
    assert cached._cached_weight is not None
    cached_loss = cached(x).float().square().mean()
    cached_loss.backward()
    flush_block_fht_weight_cache(cached)
    assert cached._cached_weight is None

    _check_close(cached_loss, dynamic_loss, dtype)
    for name in ("generator.latent", "bias", "output_gain", "input_gain"):
        got = cached.get_parameter(name).grad
        want = dynamic.get_parameter(name).grad
        assert got is not None and want is not None, name
        _check_close(got, want, dtype)


@pytest.mark.parametrize("dtype,shape_kw", [
    (F32, dict(in_features=5, out_features=3, latent_dim=8)),
    (BF16, dict(in_features=768, out_features=3072, latent_dim=32768)),
])
def test_cached_grad_matches_dynamic(dtype, shape_kw):
    """Reference tests/test_block_fht.py:78-97: no gains, bias only."""
    torch.manual_seed(123)
    dynamic = BlockFHTLinear(bias=True, layers=2, seed=11, **shape_kw).cuda().to(dtype)
    cached = BlockFHTLinear(bias=True, layers=2, seed=11, **shape_kw).cuda().to(dtype)
    cached.load_state_dict(dynamic.state_dict())
    x = torch.randn(4, dynamic.in_features, device="cuda").to(dtype)
    dynamic_loss = dynamic(x).float().square().mean()
    dynamic_loss.backward()
    prepare_block_fht_weight_cache(cached)
    cached_loss = cached(x).float().square().mean()
    cached_loss.backward()
    flush_block_fht_weight_cache(cached)
    _check_close(cached_loss, dynamic_loss, dtype)
    _check_close(cached.generator.latent.grad, dynamic.generator.latent.grad, dtype)
    _check_close(cached.bias.grad, dynamic.bias.grad, dtype)


@pytest.mark.parametrize("dtype,shape_kw", [
    (F32, dict(in_features=5, out_features=3, latent_dim=8)),
    (F32, dict(in_features=768, out_features=2304, latent_dim=17694)),
    (BF16, dict(in_features=768, out_features=3072, latent_dim=32768)),
])
def test_suspended_cache_keeps_ce_grad_and_live_perturbation_grad(dtype, shape_kw):
    """Reference tests/test_block_fht.py:146-180: a forward with a perturbed live latent runs
    between prepare and flush with the cache suspended; the flush then adds the cached (CE)
    gradient to the live perturbation gradient, as the dynamic module accumulates both."""
    from latent_weight_lab_amd import restore_block_fht_weight_cache, suspend_block_fht_weight_cache

    torch.manual_seed(456)
    dynamic = BlockFHTLinear(bias=True, layers=2, seed=17, **shape_kw).cuda().to(dtype)
    hybrid = BlockFHTLinear(bias=True, layers=2, seed=17, **shape_kw).cuda().to(dtype)
    hybrid.load_state_dict(dynamic.state_dict())
    x = torch.randn(4, dynamic.in_features, device="cuda").to(dtype)
    perturbation = torch.randn_like(dynamic.generator.latent) * 1e-3

    dynamic_base = dynamic(x).float().square().mean()
    dynamic_base.backward()
    with torch.no_grad():
        dynamic.generator.latent.add_(perturbation)
    dynamic_perturbed = dynamic(x).float().square().mean()
    dynamic_perturbed.backward()
    with torch.no_grad():
        dynamic.generator.latent.sub_(perturbation)

    prepare_block_fht_weight_cache(hybrid)
    hybrid_base = hybrid(x).float().square().mean()
    hybrid_base.backward()
    suspended = suspend_block_fht_weight_cache(hybrid)
    assert len(suspended) == 1 and hybrid._cached_weight is None
    with torch.no_grad():
        hybrid.generator.latent.add_(perturbation)
    hybrid_perturbed = hybrid(x).float().square().mean()
    hybrid_perturbed.backward()
    with torch.no_grad():
        hybrid.generator.latent.sub_(perturbation)
    restore_block_fht_weight_cache(suspended)
    assert hybrid._cached_weight is not None
    with pytest.raises(RuntimeError, match="live cached weight"):
        restore_block_fht_weight_cache(suspended)
    flush_block_fht_weight_cache(hybrid)

    _check_close(hybrid_base, dynamic_base, dtype)
    _check_close(hybrid_perturbed, dynamic_perturbed, dtype)
    _check_close(hybrid.generator.latent.grad, dynamic.generator.latent.grad, dtype)
    _check_close(hybrid.bias.grad, dynamic.bias.grad, dtype)
