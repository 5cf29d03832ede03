"""GPU parity of the HIP generator against the CPU oracle.

Bars: sign words bit-exact; float32 within 1e-5
relative L2 of the float64 oracle; bfloat16/float16 within 1e-2 relative L2
of the float32-exact result.  Full-size configs that the oracle cannot redo in
seconds are checked through size-independent properties (orthogonality per
block, adjointness, determinism) plus oracle slices.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import decode_array, gpu_available
from latent_weight_lab_amd import BlockFHT, block_fht_grad_latent, block_fht_slice
from latent_weight_lab_amd import ops
from oracle import c_oracle
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def rel_l2(got, want):
    return O.rel_l2(got, want)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()


def latent_for(n: int, seed: int, dtype=torch.float32) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g, dtype=torch.float32).to(dtype)


# ---------------------------------------------------------------- sign words

@pytest.mark.parametrize("seed,block,layer", [(7, 0, 0), (7, 255, 3), (-123456789, 2**31 + 3, 1),
                                              (2**63 - 1, 2**32 - 1, 2), (-(2**63), 17, 0)])
def test_sign_words_bit_exact(seed, block, layer):
    nwords = 1 << 18  # a 2^23 block
    got = ops.sign_words(seed, block, layer, nwords, device="cuda").cpu().numpy().view(np.uint32)
    want = O.sign_words(seed, block, layer, nwords)
    assert np.array_equal(got, want)


def test_sign_words_match_golden(golden):
    rows = golden["sign_words"]
    for seed, block, layer, word, value in rows[::7]:
        got = ops.sign_words(seed, block, layer, 1, first_word=word, device="cuda").cpu().numpy().view(np.uint32)
        assert int(got[0]) == value


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_public_signs_for(golden, dtype):
    """The public ``signs_for`` (reference block_fht.py:55-81) against the reference-written golden
    sign vectors, in the reference tensor's dtype and device, plus the reference self-test
    tests/test_block_fht.py:25-31 (signs_for == the bits of sign_word_for, position by position)."""
    from latent_weight_lab_amd import sign_word_for, signs_for

    ref = torch.empty(1, dtype=dtype, device="cuda")
    for case in golden["signs"]:
        got = signs_for(ref, case["block"], case["layer"], case["seed"], case["block_size"])
        assert got.dtype == dtype and got.device == ref.device and got.shape == (case["block_size"],)
        assert np.array_equal(to_np(got), decode_array(case["signs"])), case["seed"]
    got = signs_for(ref, block=3, layer=2, seed=999, block_size=65)
    want = [1.0 if (sign_word_for(999, 3, 2, p >> 5) >> (p & 31)) & 1 else -1.0 for p in range(65)]
    assert to_np(got).tolist() == want
    # a whole 2^15 block against the oracle's sign vector
    got = signs_for(ref, block=255, layer=3, seed=7, block_size=32768)
    assert np.array_equal(to_np(got), O.sign_vector(7, 255, 3, 32768))


# ---------------------------------------------------------------- golden fixtures

def test_golden_slices_fp32(golden):
    for case in golden["slices"]:
        latent = torch.tensor(decode_array(case["latent"]), dtype=torch.float32, device="cuda", requires_grad=True)
        args = (case["size"], case["layers"], case["seed"], case["start"], case["stop"])
        y = block_fht_slice(latent, *args)
        want = decode_array(case["out"])
        if want.size == 0:
            assert y.numel() == 0
            continue
        assert rel_l2(to_np(y), want) < 1e-5, case["name"]
        y.square().sum().backward()
        grad = to_np(latent.grad)
        if "grad_sumsq" in case:
            assert rel_l2(grad, decode_array(case["grad_sumsq"])) < 1e-5, case["name"]
        else:
            stride = case["grad_sumsq_stride"]
            assert rel_l2(grad[::stride], decode_array(case["grad_sumsq_sampled"])) < 1e-5, case["name"]


# ---------------------------------------------------------------- forward / backward sweeps

CASES = [
    # (n, size, layers, seed, start, stop)
    (1, 5, 3, 11, 0, 5),                     # B = 1
    (7, 31, 2, 123, 3, 17),                  # B = 8 (reference CPU test)
    (17, 200, 1, -4, 0, 200),                # B = 32, ragged tail
    (33, 1000, 3, 5, 63, 999),               # B = 64
    (100, 2049, 2, 2**40 + 3, 1, 2049),      # B = 128
    (300, 5000, 3, 9, 511, 4097),            # B = 512
    (1024, 108_618, 3, 123, 0, 108_618),     # config 1 full
    (1024, 108_618, 3, 123, 1000, 2000),     # config 1 slice
    (2000, 9000, 1, 77, 2047, 8193),         # B = 2048
    (4096, 8192, 1, 123, 17, 4099),          # reference smem-backend test shape
    (5000, 40000, 2, 1, 8191, 30001),        # B = 8192
    (16384, 50000, 3, 2, 0, 50000),          # B = 2^14
    (20000, 65536, 1, 123, 111, 4096),       # reference global-backend test shape (B = 2^15)
    (32768, 200_000, 3, 7, 12345, 198_765),  # B = 2^15, config-2 block size
    # more than 128 blocks: the block sum keeps 32 row loads per wave in flight, rows split
    # unevenly over its 8 waves
    (7, 1500, 2, 21, 0, 1500),               # B = 8, 188 blocks
    (32768, 150 * 32768 + 1000, 3, 13, 0, 150 * 32768 + 1000),  # B = 2^15, 151 blocks (last partial)
    (40000, 200_000, 2, 3, 1000, 150_000),   # B = 2^16: tile passes
    ((1 << 17) - 5, 300_000, 3, -9, 70_000, 299_999),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", CASES, ids=[f"n{c[0]}_s{c[1]}_L{c[2]}" for c in CASES])
def test_forward_backward_parity(case, dtype):
    n, size, layers, seed, start, stop = case
    lat = latent_for(n, n + layers, dtype)
    lat64 = lat.double().numpy()
    latent = lat.cuda().requires_grad_(True)
    y = block_fht_slice(latent, size, layers, seed, start, stop)
    assert y.dtype == dtype and y.shape == (stop - start,)
    want = c_oracle.forward(lat64, size, layers, seed, start, stop)
    assert rel_l2(to_np(y), want) < TOL[dtype]
    g = torch.randn(stop - start, generator=torch.Generator().manual_seed(1)).to(dtype)
    y.backward(g.cuda())
    gwant = c_oracle.backward(g.double().numpy(), n, size, layers, seed, start, stop)
    assert latent.grad.dtype == dtype
    assert rel_l2(to_np(latent.grad), gwant) < TOL[dtype]


def test_empty_slice_and_zero_gradient():
    latent = latent_for(64, 1).cuda().requires_grad_(True)
    y = block_fht_slice(latent, 1000, 2, 3, 500, 500)
    assert y.shape == (0,)
    g = block_fht_grad_latent(latent.detach(), torch.empty(0, device="cuda"), 1000, 2, 3, 500, 500)
    assert torch.count_nonzero(g) == 0 and g.shape == (64,)


def test_invalid_slice_raises_on_gpu():
    latent = latent_for(64, 1).cuda()
    with pytest.raises(ValueError, match="invalid slice"):
        block_fht_slice(latent, 100, 1, 0, 50, 101)
    with pytest.raises(RuntimeError, match="layers"):
        block_fht_slice(latent, 100, 0, 0, 0, 10)


# ---------------------------------------------------------------- BASELINE config 2

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_full_parity(dtype):
    """256 blocks of 2^15, layers 3, hash seed 7, latent ~N(0,1) from seed 1."""
    torch.manual_seed(1)
    lat = torch.randn(32768, dtype=torch.float32).to(dtype)
    size = 8_388_608
    latent = lat.cuda().requires_grad_(True)
    y = block_fht_slice(latent, size, 3, 7, 0, size)
    want = c_oracle.forward(lat.double().numpy(), size, 3, 7, 0, size)
    assert rel_l2(to_np(y), want) < TOL[dtype]
    g = torch.randn(size, generator=torch.Generator().manual_seed(5)).to(dtype)
    y.backward(g.cuda())
    gwant = c_oracle.backward(g.double().numpy(), 32768, size, 3, 7, 0, size)
    assert rel_l2(to_np(latent.grad), gwant) < TOL[dtype]


def test_bf16_slices_equal_full_output_bitwise():
    """A slice of the matrix-core forward is the same range of the full output, bit for
    bit, whatever its offset from the 16-byte grid (start mod 8: the slice's blocks are
    stored through shifted 16-byte slots) and wherever it starts or ends inside a block."""
    B = 32768
    size = 6 * B + 1000  # ragged last block
    lat = latent_for(B, 21, torch.bfloat16).cuda()
    full = ops.forward(lat, size, 3, 5, 0, size)
    want = c_oracle.forward(lat.double().cpu().numpy(), size, 3, 5, 0, size)
    assert rel_l2(to_np(full), want) < TOL[torch.bfloat16]
    cases = [(8 * 1000 + m, 5 * B + 77 + m) for m in range(8)]  # every grid offset, interior blocks
    cases += [(2 * B + 5, 2 * B + 100), (B - 3, B + 11), (3 * B, 4 * B), (B + 1, size), (7, 13),
              (size - 9, size)]
    for start, stop in cases:
        y = ops.forward(lat, size, 3, 5, start, stop)
        assert torch.equal(y, full[start:stop]), (start, stop)


def test_bf16_slice_backward_equals_masked_full_backward_bitwise():
    """The backward of a slice equals, bit for bit, the full backward of a gradient that is
    zero outside the slice (the same chain inputs; blocks outside add zero rows), at every
    offset of the slice's gradient from the 16-byte grid, for a fresh gradient tensor and for
    a view into a larger one."""
    B = 32768
    size = 6 * B + 1000
    n = B
    gfull = torch.randn(size, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).cuda()
    cases = [(8 * 1000 + m, 5 * B + 77 + m) for m in range(8)]
    cases += [(2 * B + 5, 2 * B + 100), (B - 3, B + 11), (B + 1, size), (size - 9, size)]
    for start, stop in cases:
        masked = torch.zeros_like(gfull)
        masked[start:stop] = gfull[start:stop]
        want = ops.backward(masked, n, torch.bfloat16, size, 3, 5, 0, size)
        for g in (gfull[start:stop].clone(), gfull[start:stop]):
            got = ops.backward(g, n, torch.bfloat16, size, 3, 5, start, stop)
            assert torch.equal(got, want), (start, stop, g.data_ptr() % 16)
    gwant = c_oracle.backward(to_np(gfull[8000:5 * B + 77]), n, size, 3, 5, 8000, 5 * B + 77)
    got = ops.backward(gfull[8000:5 * B + 77], n, torch.bfloat16, size, 3, 5, 8000, 5 * B + 77)
    assert rel_l2(to_np(got), gwant) < TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("log_block", [10, 13, 15])
def test_valu_block_paths_agree_bitwise(log_block, dtype):
    """The VALU whole-block kernels take check-free loads and stores for whole blocks and
    range-checked ones for partial blocks and short latents; all of them give the same bits:
    a latent 5 short of the block equals its zero-padded copy (forward and the gradient's
    first n values), slices equal the same range of the full output, and a slice's backward
    equals the full backward of the gradient masked to the slice."""
    B = 1 << log_block
    size = 5 * B + 1000  # ragged last block
    n = B - 5
    lat = latent_for(n, 31, dtype).cuda()
    padded = torch.cat([lat, torch.zeros(5, dtype=dtype, device="cuda")])
    full = ops.forward(lat, size, 3, 11, 0, size)
    assert torch.equal(full, ops.forward(padded, size, 3, 11, 0, size))
    want = c_oracle.forward(to_np(lat), size, 3, 11, 0, size)
    assert rel_l2(to_np(full), want) < TOL[dtype]
    for start, stop in [(7, 2 * B + 3), (B, 3 * B), (B - 1, B + 1), (3 * B + 17, size), (0, B)]:
        assert torch.equal(ops.forward(lat, size, 3, 11, start, stop), full[start:stop]), (start, stop)
    g = torch.randn(size, generator=torch.Generator().manual_seed(12)).to(dtype).cuda()
    gl = ops.backward(g, n, dtype, size, 3, 11, 0, size)
    assert torch.equal(gl, ops.backward(g, B, dtype, size, 3, 11, 0, size)[:n])
    for start, stop in [(7, 2 * B + 3), (B, 3 * B), (3 * B + 17, size)]:
        masked = torch.zeros_like(g)
        masked[start:stop] = g[start:stop]
        want = ops.backward(masked, n, dtype, size, 3, 11, 0, size)
        got = ops.backward(g[start:stop].clone(), n, dtype, size, 3, 11, start, stop)
        assert torch.equal(got, want), (start, stop)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_slice_and_determinism(dtype):
    """Config 2's slice [12,345, 1,012,345) (31 blocks, both ends inside a block) at config 2's
    own latent (seed 1) and hash seed 7: forward and backward against the C oracle, and
    run-to-run bit equality of both (the block sum runs in a fixed order)."""
    torch.manual_seed(1)
    lat = torch.randn(32768, dtype=torch.float32).to(dtype)
    start, stop = 12_345, 1_012_345
    latent = lat.cuda()
    y1 = ops.forward(latent, 8_388_608, 3, 7, start, stop)
    y2 = ops.forward(latent, 8_388_608, 3, 7, start, stop)
    assert torch.equal(y1, y2)
    want = c_oracle.forward(lat.double().numpy(), 8_388_608, 3, 7, start, stop)
    assert rel_l2(to_np(y1), want) < TOL[dtype]
    g = torch.randn(stop - start, generator=torch.Generator().manual_seed(2)).to(dtype)
    b1 = ops.backward(g.cuda(), 32768, dtype, 8_388_608, 3, 7, start, stop)
    b2 = ops.backward(g.cuda(), 32768, dtype, 8_388_608, 3, 7, start, stop)
    assert torch.equal(b1, b2)  # fixed-order reduction
    gwant = c_oracle.backward(g.double().numpy(), 32768, 8_388_608, 3, 7, start, stop)
    assert rel_l2(to_np(b1), gwant) < TOL[dtype]


# ---------------------------------------------------------------- BASELINE config 3 (multi-pass)

@pytest.mark.parametrize("log_block", [20, 23])
def test_config3_multipass(log_block):
    """size 2^26, fp32, layers 3, hash seed 99, latent ~N(0,1) from seed 2."""
    B = 1 << log_block
    size = 1 << 26
    torch.manual_seed(2)
    lat = torch.randn(B, dtype=torch.float32)
    latent = lat.cuda()
    y = ops.forward(latent, size, 3, 99, 0, size)
    # every block is an orthogonal image of the latent
    norms = y.view(-1, B).double().norm(dim=1).cpu().numpy()
    assert np.allclose(norms, float(lat.double().norm()), rtol=1e-5)
    # oracle on a slice straddling blocks 1|2 and on the last block
    for s0, s1 in [(2 * B - 777, 2 * B + 4321), (size - B, size)]:
        want = c_oracle.forward(lat.double().numpy(), size, 3, 99, s0, s1)
        assert rel_l2(to_np(y[s0:s1]), want) < 1e-5
    # the forward runs its passes over groups of blocks of at most 128 MiB of float32 work
    # (32 blocks of 2^20, 4 of 2^23): a slice over more than one group, partial at both ends,
    # equals the full call bit for bit, and the oracle around its ends and the group boundary
    per = (128 << 20) // (4 * B)
    s0, s1 = 12345, (per + 2) * B + 999
    ys = ops.forward(latent, size, 3, 99, s0, s1)
    assert torch.equal(ys, y[s0:s1])
    for w0, w1 in [(s0, s0 + 3000), (per * B - 1500, per * B + 1500), (s1 - 3000, s1)]:
        want = c_oracle.forward(lat.double().numpy(), size, 3, 99, w0, w1)
        assert rel_l2(to_np(ys[w0 - s0:w1 - s0]), want) < 1e-5
    # adjointness <T x, g> = <x, T^T g> over the full size (fp64 dot products)
    g = torch.randn(size, generator=torch.Generator().manual_seed(3)).cuda()
    gl = ops.backward(g, B, torch.float32, size, 3, 99, 0, size)
    lhs = float(torch.dot(y.double(), g.double()))
    rhs = float(torch.dot(latent.double(), gl.double()))
    scale = float(y.double().norm() * g.double().norm())
    assert abs(lhs - rhs) < 1e-6 * scale
    # backward of one block vs the oracle
    s0, s1 = 3 * B, 4 * B
    gwant = c_oracle.backward(g[s0:s1].double().cpu().numpy(), B, size, 3, 99, s0, s1)
    gb = ops.backward(g[s0:s1].contiguous(), B, torch.float32, size, 3, 99, s0, s1)
    assert rel_l2(to_np(gb), gwant) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layers", [1, 2, 3])
@pytest.mark.parametrize("log_block", [16, 17, 18, 19, 20, 21, 22, 23])
def test_tile_pass_block_sizes(log_block, layers, dtype):
    """Every multi-pass block size: the tile passes' bit groups depend on it (tiles of up
    to 2^20 blocks stay in registers, larger ones send a 1-3 bit group through LDS), and
    the layer count decides which passes transform before or after their sign layer.
    Forward and backward on a ragged size and a slice across two block boundaries."""
    B = 1 << log_block
    n = B - 3
    size = 2 * B + B // 2 + 7
    lat = latent_for(n, log_block + layers, dtype)
    latent = lat.cuda()
    s0, s1 = B - 1000, 2 * B + 1234
    y = ops.forward(latent, size, layers, 17, s0, s1)
    assert y.dtype == dtype
    want = c_oracle.forward(lat.double().numpy(), size, layers, 17, s0, s1)
    assert rel_l2(to_np(y), want) < TOL[dtype]
    g = torch.randn(s1 - s0, generator=torch.Generator().manual_seed(log_block)).to(dtype).cuda()
    gl = ops.backward(g, n, dtype, size, layers, 17, s0, s1)
    gwant = c_oracle.backward(g.double().cpu().numpy(), n, size, layers, 17, s0, s1)
    assert rel_l2(to_np(gl), gwant) < TOL[dtype]


@pytest.mark.parametrize("log_block,nblocks,layers,dtype", [
    (16, 301, 3, torch.float32),    # 2 tiles per block: 101 groups of 3 blocks, the last of 1, then the group sum
    (21, 13, 2, torch.bfloat16),    # 64 tiles per block: 4 groups of 4, the last of 1; even L ends on a low pass
    (22, 3, 1, torch.float32),      # 128 tiles per block: one group, summed straight into grad_latent
])
def test_tile_pass_grouped_block_sum(log_block, nblocks, layers, dtype):
    """The backward's last tile pass sums the blocks: workgroup (tile, group) adds one tile's
    positions over a group of blocks in ascending order, with more than one group a block sum
    over the groups' rows follows.  Full-size backward against the C oracle, reruns bit-identical."""
    B = 1 << log_block
    n = B - 5
    size = nblocks * B - 11
    g = torch.randn(size, generator=torch.Generator().manual_seed(nblocks)).to(dtype)
    gd = g.cuda()
    gl = ops.backward(gd, n, dtype, size, layers, 31, 0, size)
    gl2 = ops.backward(gd, n, dtype, size, layers, 31, 0, size)
    torch.cuda.synchronize()
    assert torch.equal(gl, gl2)
    gwant = c_oracle.backward(g.double().numpy(), n, size, layers, 31, 0, size)
    assert rel_l2(to_np(gl), gwant) < TOL[dtype]


def test_reference_2_23_smoke():
    # reference tests/test_block_fht_cuda.py:34-40
    bfht = BlockFHT((1 << 23) - 17, size=1 << 23, layers=1, seed=9).cuda()
    out = bfht.slice(12345, 12345 + 1024)
    out.square().mean().backward()
    torch.cuda.synchronize()
    assert out.shape == (1024,)
    assert bfht.latent.grad is not None and torch.isfinite(bfht.latent.grad).all()
    lat = bfht.latent.detach().double().cpu().numpy()
    want = c_oracle.forward(lat, 1 << 23, 1, 9, 12345, 12345 + 1024)
    assert rel_l2(to_np(out), want) < 1e-5
