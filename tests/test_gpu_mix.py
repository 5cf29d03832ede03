"""GPU parity of the signed activation FHT (``FixedFHTMix``, reference
``examples/nanogpt/model.py:200-218``) against the oracle's restatement
(``oracle.fixed_fht_mix``, pinned by the dense signed Hadamard product).

Bar: float32 1e-5, bf16 / fp16 1e-2 relative L2 (the kernel computes in float32
and rounds once; the reference's torch loop rounds at every stage in the
activation dtype).
"""
from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import FixedFHTMix, fixed_fht_mix
from latent_weight_lab_amd import ops
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def signs_for(P, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 2, (P,), generator=g, dtype=torch.float32) * 2.0 - 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,features", [(4096, 768), (300, 3072), (7, 1), (33, 5), (64, 32), (65, 33),
                                           (10, 1000), (9, 4096), (3, 32768), (1, 20000),
                                           # one-wave rows (P = 1024, 4096): odd row counts, ragged
                                           # rows and rows of no whole 16-byte chunks
                                           (7, 1000), (3, 517), (5, 2051), (129, 4000)])
def test_mix_matches_oracle(rows, features, dtype):
    P = ops.next_power_of_two(features)
    s = signs_for(P, features)
    x = torch.randn(rows, features, generator=torch.Generator().manual_seed(rows)).to(dtype)
    got = ops.fht_mix(x.cuda(), s.cuda())
    torch.cuda.synchronize()
    want = O.fixed_fht_mix(x.double().numpy(), s.double().numpy())
    assert got.dtype == dtype and got.shape == x.shape
    assert O.rel_l2(got.double().cpu().numpy(), want) < TOL[dtype]


def test_mix_in_place_and_empty():
    for rows, features, P in ((100, 768, 1024), (37, 3072, 4096), (11, 1500, 2048)):
        s = signs_for(P, 1).cuda()
        x = torch.randn(rows, features, device="cuda")
        want = ops.fht_mix(x, s)
        ops.fht_mix(x, s, out=x)
        assert torch.equal(x, want)
    e = torch.empty(0, 768, device="cuda")
    assert ops.fht_mix(e, signs_for(1024, 1).cuda()).shape == (0, 768)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,features", [(101, 768), (3, 1000), (37, 3072), (5, 4096),
                                           # more row groups than the launch's waves: each wave loops
                                           (9001, 768), (5000, 3072)])
def test_mix_matrix_core_rows(rows, features, dtype):
    """The matrix-core kernel (bf16 / fp16 rows of P = 1024 and 4096; four rows per wave at
    1024, a row count that is no multiple of four leaves the last wave's rows partly empty):
    against the oracle, and in place equal to out of place bit for bit."""
    P = ops.next_power_of_two(features)
    s = signs_for(P, rows + features)
    x = torch.randn(rows, features, generator=torch.Generator().manual_seed(rows)).to(dtype).cuda()
    got = ops.fht_mix(x, s.cuda())
    y = x.clone()
    ops.fht_mix(y, s.cuda(), out=y)
    torch.cuda.synchronize()
    assert torch.equal(y, got)
    want = O.fixed_fht_mix(x.double().cpu().numpy(), s.double().numpy())
    assert O.rel_l2(got.double().cpu().numpy(), want) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,features", [(9, 3072), (6, 768)])
def test_mix_unaligned_buffers(rows, features, dtype):
    """x and out one element off the 16-byte grid: the element-store paths, equal to the
    aligned call bit for bit."""
    P = ops.next_power_of_two(features)
    s = signs_for(P, 4).cuda()
    x = torch.randn(rows, features, generator=torch.Generator().manual_seed(7)).to(dtype).cuda()
    want = ops.fht_mix(x, s)
    xb = torch.zeros(rows * features + 1, dtype=dtype, device="cuda")
    xb[1:] = x.reshape(-1)
    ob = torch.zeros(rows * features + 2, dtype=dtype, device="cuda")
    xv = xb[1:].view(rows, features)
    ov = ob[1:-1].view(rows, features)
    assert xv.data_ptr() % 16 != 0 and ov.data_ptr() % 16 != 0
    ops.fht_mix(xv, s, out=ov)
    torch.cuda.synchronize()
    assert torch.equal(ov, want)
    assert ob[0].item() == 0 and ob[-1].item() == 0  # nothing written outside out


def test_mix_involution_at_power_of_two():
    s = signs_for(4096, 2).cuda()
    x = torch.randn(50, 4096, device="cuda")
    back = ops.fht_mix(ops.fht_mix(x, s), s)
    assert O.rel_l2(back.double().cpu().numpy(), x.double().cpu().numpy()) < 1e-6


def test_module_forward_and_backward():
    mix = FixedFHTMix(768, 1000 + 66).cuda()
    ref_signs = torch.randint(0, 2, (1024,), generator=torch.Generator().manual_seed(1066),
                              dtype=torch.float32) * 2.0 - 1.0
    assert torch.equal(mix.signs.cpu(), ref_signs)  # the reference's buffer recipe
    x = torch.randn(2, 10, 768, device="cuda", requires_grad=True)
    g = torch.randn(2, 10, 768, device="cuda")
    y = mix(x)
    (y * g).sum().backward()
    s = ref_signs.double().numpy()
    assert O.rel_l2(y.detach().double().cpu().numpy(), O.fixed_fht_mix(x.detach().double().cpu().numpy(), s)) < 1e-5
    # the map is symmetric: d<y, g>/dx = mix(g)
    assert O.rel_l2(x.grad.double().cpu().numpy(), O.fixed_fht_mix(g.double().cpu().numpy(), s)) < 1e-5
    with pytest.raises(ValueError):
        mix(torch.randn(3, 767, device="cuda"))


def test_functional_bf16_grad():
    s = signs_for(4096, 3).cuda()
    x = torch.randn(64, 3072, device="cuda").to(torch.bfloat16).requires_grad_(True)
    y = fixed_fht_mix(x, s)
    y.float().sum().backward()
    ones = torch.ones(64, 3072)
    want = O.fixed_fht_mix(ones.double().numpy(), s.double().cpu().numpy())
    assert x.grad.dtype == torch.bfloat16
    assert O.rel_l2(x.grad.double().cpu().numpy(), want) < 1e-2
