"""GPU tests of BlockFHTLinear's spectral correction: W' = (W + U C V^T) * exp(g_out) (x) exp(g_in),
with U, V fixed Walsh columns and C, g_out, g_in trained (reference
latent_weight_lab/block_fht.py:405-414 (construction), :426-435 (_hadamard_columns),
:452-458 (weight), :503-505 (no weight cache); tests/test_block_fht.py:208-229).

The reference tests run on the CPU in float32 at one tiny shape; here the module runs on the
GPU in float32 and bfloat16, at the reference's shape and at a GPT-2 MLP shape whose
bf16 latent of 2^15 takes the matrix-core generator.  Gradients are checked against a
float64 autograd composition built on the C oracle's generated weight and, for the latent,
the oracle's adjoint (float32 1e-5, bfloat16 1e-2 relative L2).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import BlockFHTLinear
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

F32, BF16 = torch.float32, torch.bfloat16
TOL = {F32: 1e-5, BF16: 1e-2}
SPECTRAL = ("spectral_u", "spectral_v", "spectral_core", "spectral_log_out_gain", "spectral_log_in_gain")

# (in, out, latent_dim, layers, seed, rank, out_groups, in_groups, tokens)
SHAPES = [
    (8, 12, 8, 2, 9, 2, 3, 2, 4),                   # the reference tests' shape
    (768, 3072, 32768, 3, 5, 4, 4, 3, 64),          # GPT-2 MLP, block 2^15 (matrix cores in bf16)
]


def rel(got, want):
    return O.rel_l2(np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64))


def module(shape, dtype, spectral=True, bias=True):
    fin, fout, ld, layers, seed, rank, og, ig, _ = shape
    kw = dict(spectral_rank=rank, spectral_out_groups=og, spectral_in_groups=ig) if spectral else {}
    torch.manual_seed(seed)
    return BlockFHTLinear(fin, fout, bias=bias, latent_dim=ld, layers=layers, seed=seed, **kw).to(dtype).cuda()


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("shape", SHAPES, ids=["ref_8x12", "gpt2_768x3072"])
def test_spectral_zero_correction_matches_same_seed_base(shape, dtype):
    """Reference tests/test_block_fht.py:208-215: a spectral module loaded from a plain
    module's state dict (its spectral parameters left at their zero / unit start) has the
    plain module's weight and output."""
    base = module(shape, dtype, spectral=False)
    structured = module(shape, dtype)
    missing, unexpected = structured.load_state_dict(base.state_dict(), strict=False)
    assert not unexpected and set(missing) == set(SPECTRAL)
    x = torch.randn(shape[-1], shape[0], generator=torch.Generator().manual_seed(1)).to(dtype).cuda()
    with torch.no_grad():
        w_base, w_struct = base.weight, structured.weight
        assert torch.equal(w_struct, w_base)  # + U 0 V^T and * exp(0) change no bit
        y_base, y_struct = base(x), structured(x)
    torch.cuda.synchronize()
    assert rel(y_struct.float().cpu(), y_base.float().cpu()) <= TOL[dtype]


def composition(layer, x, dt, weight_scale=1.0):
    """Loss mean((x W'^T + b)^2) on the CPU in dtype dt from the C oracle's generated weight
    (rounded to the module's dtype, as the generator's output is) and the module's parameters,
    with gradients of C, g_out, g_in, the bias and W (in float64, the latter projected onto the
    latent by the oracle's adjoint)."""
    g = layer.generator
    lat = g.latent.detach().double().cpu().numpy()
    size = layer.in_features * layer.out_features
    w0 = torch.tensor(c_oracle.forward(lat, size, g.layers, g.seed, 0, size) * weight_scale,
                      dtype=torch.float64).view(layer.out_features, layer.in_features)
    if dt != torch.float64:
        w0 = w0.to(layer.spectral_core.dtype).to(dt)
    w0.requires_grad_(True)
    d = lambda t: t.detach().cpu().to(dt).requires_grad_(True)  # noqa: E731
    core, lo, li = d(layer.spectral_core), d(layer.spectral_log_out_gain), d(layer.spectral_log_in_gain)
    bias = d(layer.bias)
    u, v = layer.spectral_u.cpu().to(dt), layer.spectral_v.cpu().to(dt)
    out_gain = lo.exp().repeat_interleave(layer.out_features // layer.spectral_out_groups)
    in_gain = li.exp().repeat_interleave(layer.in_features // layer.spectral_in_groups)
    w = (w0 + u @ core @ v.t()) * out_gain.view(-1, 1) * in_gain.view(1, -1)
    y = torch.nn.functional.linear(x.cpu().to(dt), w, bias)
    (y if dt == torch.float64 else y.float()).square().mean().backward()
    res = {"spectral_core": core.grad, "spectral_log_out_gain": lo.grad, "spectral_log_in_gain": li.grad,
           "bias": bias.grad}
    if dt == torch.float64:
        res["latent"] = c_oracle.backward(w0.grad.numpy().reshape(-1) * weight_scale, g.latent.numel(), size,
                                          g.layers, g.seed, 0, size)
    return res


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("shape", SHAPES, ids=["ref_8x12", "gpt2_768x3072"])
def test_spectral_core_and_gains_get_gradients_and_no_cache(shape, dtype):
    """Reference tests/test_block_fht.py:217-229: with a nonzero core, the weight cache stays
    empty and the core, both group gains, the bias and the latent receive finite gradients —
    here also equal to the float64 composition's."""
    layer = module(shape, dtype)
    gen = torch.Generator().manual_seed(2)
    with torch.no_grad():
        layer.spectral_core.copy_(0.1 * torch.randn(layer.spectral_core.shape, generator=gen))
        layer.spectral_log_out_gain.copy_(0.2 * torch.randn(layer.spectral_log_out_gain.shape, generator=gen))
        layer.spectral_log_in_gain.copy_(0.2 * torch.randn(layer.spectral_log_in_gain.shape, generator=gen))
        # a bias and inputs with components along the Walsh columns: with random ones the
        # 4 x 4 projection U^T (dL/dW) V is a sum of ~10^6 terms that cancel to far below their
        # size, and bfloat16's rounding of dL/dW (torch's ops) then dominates the core gradient
        rank = layer.spectral_rank
        u, v = layer.spectral_u.float().cpu(), layer.spectral_v.float().cpu()
        bias = 0.1 * torch.randn(layer.out_features, generator=gen)
        bias += (u * layer.out_features ** 0.5) @ torch.randn(rank, generator=gen)
        layer.bias.copy_(bias)
    layer.materialize_weight_cache()
    assert layer._cached_weight is None
    x = torch.randn(shape[-1], shape[0], generator=gen)
    x += torch.randn(shape[-1], rank, generator=gen) @ (v * layer.in_features ** 0.5).t()
    x = x.to(dtype).cuda()
    layer(x).float().square().mean().backward()
    torch.cuda.synchronize()
    want = composition(layer, x, torch.float64)
    got = {"spectral_core": layer.spectral_core.grad, "spectral_log_out_gain": layer.spectral_log_out_gain.grad,
           "spectral_log_in_gain": layer.spectral_log_in_gain.grad, "bias": layer.bias.grad,
           "latent": layer.generator.latent.grad}
    err = lambda a, b: rel(np.asarray(a.float().cpu() if torch.is_tensor(a) else a).reshape(-1),  # noqa: E731
                           np.asarray(b, dtype=np.float64).reshape(-1))
    # The spectral terms are torch ops in the module's dtype (as in the reference): in bfloat16
    # their bar is also at most twice the error of the same ops on the CPU (torch's bfloat16
    # arithmetic alone: ~1.1e-2 for the core at the GPT-2 shape, whose 4 x 4 Walsh projection of
    # dL/dW cancels); the latent's gradient runs through the library's backward: 1e-2.
    tol = dict.fromkeys(got, TOL[dtype])
    if dtype != F32:
        ref_dt = composition(layer, x, dtype)
        for name, g in ref_dt.items():
            tol[name] = max(tol[name], 2 * err(g, want[name]))
    errs = {}
    for name, g in got.items():
        assert g is not None and torch.isfinite(g).all(), name
        errs[name] = err(g, want[name])
    print(f"{shape[:2]} {dtype}: " + ", ".join(f"{k} {v:.2e} (bar {tol[k]:.1e})" for k, v in errs.items()))
    assert all(errs[k] <= tol[k] for k in errs), errs
    for p in (layer.spectral_core, layer.spectral_log_out_gain, layer.spectral_log_in_gain):
        assert p.requires_grad

