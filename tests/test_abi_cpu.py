"""CPU-only checks of the C ABI: the library loads beside torch, exports every
declared symbol, shares torch's HIP runtime, and validates arguments with the
reference's messages — without launching anything."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (must precede the library: it owns the HIP runtime)

from latent_weight_lab_amd import _native as N
from latent_weight_lab_amd import ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "lwl_bfht.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lwl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name


def test_library_shares_torch_hip_runtime():
    N.lib()
    maps = Path("/proc/self/maps").read_text()
    hip_paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(hip_paths) == 1, hip_paths
    assert "torch" in next(iter(hip_paths))


def test_abi_version():
    assert N.lib().lwl_abi_version() == 2


@pytest.mark.parametrize(
    "args, code, msg",
    [
        ((0, 1024, 108_618, 3, 1000, 2000), N.LWL_OK, ""),
        ((2, 1, 5, 1, 0, 5), N.LWL_OK, ""),                     # B = 1 is accepted
        ((0, 1024, 100, 3, 50, 200), N.LWL_ERR_INVALID, "invalid slice [50, 200) for size 100"),
        ((0, 1024, 100, 3, 60, 50), N.LWL_ERR_INVALID, "invalid slice [60, 50) for size 100"),
        ((0, 1024, 100, 3, -1, 5), N.LWL_ERR_INVALID, "invalid slice"),
        ((0, 1024, 100, 0, 0, 5), N.LWL_ERR_INVALID, "layers must be 1, 2, or 3"),
        ((0, 1024, 100, 4, 0, 5), N.LWL_ERR_INVALID, "layers must be 1, 2, or 3"),
        ((0, 0, 100, 1, 0, 5), N.LWL_ERR_INVALID, "latent size must be positive"),
        ((0, 10, 0, 1, 0, 0), N.LWL_ERR_INVALID, "size must be positive"),
        ((0, (1 << 23) + 1, 1 << 24, 1, 0, 5), N.LWL_ERR_UNSUPPORTED, "2^23"),
        ((7, 16, 100, 1, 0, 5), N.LWL_ERR_UNSUPPORTED, "float32, float16 and bfloat16"),
    ],
)
def test_forward_validation(args, code, msg):
    lib = N.lib()
    assert lib.lwl_bfht_check_forward(*args) == code
    assert msg in lib.lwl_last_error().decode()


def test_invalid_argument_maps_to_value_and_runtime_error():
    lib = N.lib()
    rc = lib.lwl_bfht_check_forward(0, 16, 10, 1, 5, 11)
    with pytest.raises(ValueError, match="invalid slice"):
        N.check(rc)
    rc = lib.lwl_bfht_check_forward(0, 16, 10, 1, 5, 11)
    with pytest.raises(RuntimeError, match="invalid slice"):
        N.check(rc)


def test_forward_rejects_missing_workspace_without_launching():
    lib = N.lib()
    # B = 2^20 needs a work buffer; a null workspace must fail before any launch
    rc = lib.lwl_bfht_forward(1, 0, 1 << 20, 1 << 21, 1, 0, 0, 10, 1, 0, 0, 0)
    assert rc == N.LWL_ERR_WORKSPACE
    assert "workspace" in lib.lwl_last_error().decode()


def test_workspace_sizes():
    lib = N.lib()
    assert lib.lwl_bfht_forward_workspace_size(32768, 8 << 20, 0, 8 << 20) == 0
    # the tile-pass forward works through groups of blocks of at most 128 MiB of float32
    assert lib.lwl_bfht_forward_workspace_size(1 << 20, 1 << 26, 0, 1 << 26) == 32 * (1 << 20) * 4
    assert lib.lwl_bfht_forward_workspace_size(1 << 23, 1 << 26, 0, 1 << 26) == 4 * (1 << 23) * 4
    assert lib.lwl_bfht_forward_workspace_size(1 << 16, 1 << 20, 0, 1 << 20) == 16 * (1 << 16) * 4
    # slice [12345, 1012345) of B=2^20 touches blocks 0..0
    assert lib.lwl_bfht_forward_workspace_size(1 << 20, 1 << 26, 12345, 1_012_345) == (1 << 20) * 4
    # backward whole-block sizes: one float32 partial row of latent_size per overlapped block,
    # at least one 8-value bfloat16 row (16 bytes) for the matrix-core chain's padded rows
    assert lib.lwl_bfht_backward_workspace_size(1024, 108_618, 1000, 2000) == 2 * 1024 * 4
    assert lib.lwl_bfht_backward_workspace_size(3, 4096, 0, 4096) == 1024 * 16
    assert lib.lwl_bfht_backward_workspace_size(5, 4096, 0, 4096) == 512 * 20
    assert lib.lwl_bfht_backward_workspace_size(1024, 108_618, 0, 1024) == 1024 * 4
    assert lib.lwl_bfht_backward_workspace_size(32768, 8 << 20, 0, 8 << 20) == 256 * 32768 * 4
    assert lib.lwl_bfht_backward_workspace_size(16, 40, 3, 3) == 0
    assert lib.lwl_bfht_backward_workspace_size(1 << 23, 1 << 26, 0, 1 << 26) == 8 * (1 << 23) * 4


def test_noalloc_backward_refuses_oversized_scratch_on_the_host():
    """lwl_bfht_backward_noalloc refuses a call whose scratch exceeds its 32 MiB device array
    before any HIP call: config 3 at 2^20 needs a 256 MiB work buffer.  The pointers are fake
    (never dereferenced); were the guard to let the call through, it would fail here with a
    HIP error (no device), not touch memory."""
    lib = N.lib()
    need = lib.lwl_bfht_backward_workspace_size(1 << 20, 1 << 26, 0, 1 << 26)
    assert need > 32 << 20
    rc = lib.lwl_bfht_backward_noalloc(0x10000, 0, 1 << 20, 1 << 26, 3, 99, 0, 1 << 26, 0x20000, None)
    assert rc == N.LWL_ERR_UNSUPPORTED
    msg = lib.lwl_last_error().decode()
    assert "bytes of scratch" in msg and str(need) in msg


def test_cpu_tensors_fail_loudly():
    from latent_weight_lab_amd import BlockFHT

    bfht = BlockFHT(16, size=40, layers=1, seed=1)
    with pytest.raises(RuntimeError, match="GPU"):
        bfht()


def test_module_metadata_and_validation():
    from latent_weight_lab_amd import BlockFHT, BlockFHTLinear

    # reference tests/test_block_fht.py:49-59
    latent = torch.nn.Parameter(torch.randn(8))
    assert BlockFHT(latent, size=40, layers=1, seed=5).latent is latent
    assert BlockFHT(32, size=64, layers=1, seed=1).block_size == 32
    assert BlockFHT((1 << 23) - 17, size=1 << 23, layers=1, seed=1).block_size == 1 << 23
    with pytest.raises(ValueError):
        BlockFHT(8, size=0)
    with pytest.raises(ValueError):
        BlockFHT(8, size=10, layers=4)
    with pytest.raises(ValueError):
        BlockFHT(torch.zeros(2, 2), size=10)
    layer = BlockFHTLinear(768, 3072, latent_dim=32768, layers=3, seed=3)
    assert layer.generator.block_size == 32768 and layer.generator.size == 768 * 3072


@pytest.mark.parametrize("fin,fout,seed,rank", [(8, 12, 9, 2), (768, 3072, 5, 4), (5, 7, -40, 3)])
def test_spectral_buffers_are_persistent_walsh_columns(fin, fout, seed, rank):
    """BlockFHTLinear's spectral_u / spectral_v (reference block_fht.py:411-412,426-435) travel
    in the state dict and hold columns seed + 17 .. and seed + 31 .. of the order-n Sylvester
    matrix over sqrt(n): entry (i, j) = (-1)^popcount(i & (first + j)) / sqrt(n), rows 0 .. n-1
    (n need not be a power of two: the rows are truncated)."""
    import math

    import numpy as np

    from latent_weight_lab_amd import BlockFHTLinear

    layer = BlockFHTLinear(fin, fout, latent_dim=8, layers=2, seed=seed, spectral_rank=rank)
    sd = layer.state_dict()
    for name, n, first in (("spectral_u", fout, seed + 17), ("spectral_v", fin, seed + 31)):
        assert name in sd
        cols = [first + j for j in range(rank)]
        # negative column indices (seed < -31) follow the two's-complement int64 AND
        signs = [[1.0 - 2.0 * (bin((i & c) & ((1 << 64) - 1)).count("1") & 1) for c in cols] for i in range(n)]
        # the reference divides the float32 signs by the Python float sqrt(n) (block_fht.py:435)
        want = torch.tensor(signs, dtype=torch.float32) / math.sqrt(n)
        assert torch.equal(sd[name], want), name
        assert np.allclose(sd[name].double().numpy(), np.array(signs) / np.sqrt(n), rtol=1e-7, atol=0), name


def test_sign_word_api_matches_oracle():
    from latent_weight_lab_amd import sign_word_for
    from oracle import oracle as O

    for args in [(999, 3, 2, 4), (-1, 0, 0, 0), (2**63 - 1, 2**32 - 1, 3, 262143), (-(2**63), 5, 1, 7)]:
        assert sign_word_for(*args) == O.sign_word_for(*args)


def test_next_power_of_two():
    assert [ops.next_power_of_two(v) for v in (1, 2, 3, 1024, 1025, 20000)] == [1, 2, 4, 1024, 2048, 32768]
    with pytest.raises(ValueError):
        ops.next_power_of_two(0)


@pytest.mark.parametrize(
    "args, code, msg",
    [
        # (dtype, tokens, in_features, latent_size, out_features, layers)
        ((2, 4096, 768, 32768, 3072, 3), N.LWL_OK, ""),           # GPT-2 MLP up, bf16: fused
        ((2, 4096, 3072, 32768, 768, 3), N.LWL_OK, ""),           # GPT-2 MLP down
        ((2, 1, 1000, 30000, 77, 2), N.LWL_OK, ""),               # rows straddle blocks
        ((0, 16, 768, 32768, 3072, 3), N.LWL_ERR_UNSUPPORTED, "bfloat16"),  # fp32: generate + F.linear
        ((2, 16, 768, 16384, 3072, 3), N.LWL_ERR_UNSUPPORTED, "bfloat16"),  # block 2^14
        ((2, 16, 100, 32768, 30, 3), N.LWL_ERR_UNSUPPORTED, "in_features"),  # in % 8 != 0, >64 rows
        ((2, 16, 40000, 32768, 3, 3), N.LWL_ERR_UNSUPPORTED, "block_size"),  # in > B
        ((2, 16, 520, 32768, 64, 3), N.LWL_ERR_UNSUPPORTED, "528 <= in_features <= 5120"),  # > 64 rows per block
        ((2, 16, 528, 32768, 64, 3), N.LWL_OK, ""),                # 62 rows + 2 partial: 4 row tiles
        ((2, 16, 5120, 32768, 64, 3), N.LWL_OK, ""),               # largest k-major table (160 KiB)
        ((2, 16, 5128, 32768, 64, 3), N.LWL_ERR_UNSUPPORTED, "528 <= in_features <= 5120"),  # table too big
        ((2, 16, 768, 32768, 3072, 4), N.LWL_ERR_INVALID, "layers must be 1, 2, or 3"),
        ((2, 16, 0, 32768, 3072, 3), N.LWL_ERR_INVALID, "in_features must be positive"),
        ((2, 1 << 20, 1024, 32768, 64, 3), N.LWL_ERR_UNSUPPORTED, "2^30"),
        ((2, 16, 768, 32768, 1 << 26, 3), N.LWL_ERR_UNSUPPORTED, "2^26"),       # 16 tokens' rows of out > 2 GiB
        ((2, 16, 5120, 32768, 1 << 20, 3), N.LWL_ERR_UNSUPPORTED, "2^31"),      # > 65536 tile boundaries
        # the reference extension's own domain (block <= 2^14, block % in == 0), every dtype
        ((0, 5, 8, 32, 6, 2), N.LWL_OK, ""),                                   # reference test shape
        ((1, 1, 1024, 16384, 4096, 2), N.LWL_OK, ""),                          # reference profiling case
        ((2, 300, 1024, 16384, 4096, 3), N.LWL_OK, ""),
        ((0, 9, 1, 1, 7, 3), N.LWL_OK, ""),                                    # block 2^0
        ((0, 16, 768, 16384, 3072, 3), N.LWL_ERR_UNSUPPORTED, "block_size % in_features == 0"),
        ((0, 1 << 20, 1024, 16384, 4096, 2), N.LWL_ERR_UNSUPPORTED, "2 GiB"),   # tokens * out * 4 >= 2^31
    ],
)
def test_linear_validation(args, code, msg):
    lib = N.lib()
    assert lib.lwl_bfht_check_linear_forward(*args) == code
    if msg:
        assert msg in lib.lwl_last_error().decode()


def test_linear_workspace_size():
    # one pair of float32 partial rows (first / last row of the tile) per workgroup tile of generated
    # blocks and token, then, from 256 tokens, x re-laid out in 16-token x 32-k tiles of 1 KiB
    # (zero-padded).  From 256 tokens a tile is two blocks when one block holds at most 64 rows and
    # two fit in the LDS (here: 1000 in_features, 67 rows at an exact pitch; 3072 below 2048
    # tokens, test_linear_workspace_three_block_tiles); otherwise, and below, one block.  Rows of
    # 768 take tiles of 64 whole rows instead (1.5 blocks): no row straddles two tiles, so no
    # partial rows, only the x copy.
    lib = N.lib()
    assert lib.lwl_bfht_linear_forward_workspace_size(4096, 768, 3072, 32768) == 256 * 24 * 1024
    partial = (18 * 2 * 255 * 4 + 255) // 256 * 256
    assert lib.lwl_bfht_linear_forward_workspace_size(255, 768, 768, 32768) == partial
    partial = (7 * 2 * 300 * 4 + 255) // 256 * 256
    assert lib.lwl_bfht_linear_forward_workspace_size(300, 1000, 450, 32768) == partial + 19 * 32 * 1024
    # 528 in_features: 125 rows per two blocks exceed the register budget: one block per tile
    partial = (ceil_div(528 * 100, 32768) * 2 * 300 * 4 + 255) // 256 * 256
    assert lib.lwl_bfht_linear_forward_workspace_size(300, 528, 100, 32768) == partial + 19 * 17 * 1024
    # the reference-domain kernels (block <= 2^14) keep W in LDS; from 256 tokens the matrix-core
    # one reads x from a copy in MFMA order: ceil(tokens / 16) tiles x (in * 4 bytes / 64) steps of
    # 1 KiB for float32, the largest of the dtypes (the query has none)
    assert lib.lwl_bfht_linear_forward_workspace_size(5, 8, 6, 32) == 0
    assert lib.lwl_bfht_linear_forward_workspace_size(255, 1024, 4096, 16384) == 0
    assert lib.lwl_bfht_linear_forward_workspace_size(300, 1024, 4096, 16384) == 19 * 64 * 1024
    assert lib.lwl_bfht_linear_forward_ex_workspace_size(1, 300, 1024, 4096, 16384, None) == 19 * 32 * 1024


def ceil_div(a, b):
    return -(-a // b)

@pytest.mark.parametrize(
    "args,code,msg",
    [
        # (dtype, tokens, in_features, latent_size, out_features, layers)
        ((2, 4096, 768, 32768, 3072, 3), N.LWL_OK, ""),
        ((2, 4096, 3072, 32768, 768, 3), N.LWL_OK, ""),
        ((2, 0, 768, 32768, 3072, 3), N.LWL_OK, ""),
        ((0, 16, 768, 32768, 3072, 3), N.LWL_ERR_UNSUPPORTED, "bfloat16"),     # fp32: grad_weight in HBM
        ((2, 16, 520, 32768, 64, 3), N.LWL_OK, ""),                          # any in_features
        ((2, 16, 77, 32768, 33, 3), N.LWL_OK, ""),                           # rows off the 16-byte grid
        ((2, 16, 768, 8192, 64, 3), N.LWL_ERR_UNSUPPORTED, "block 2^15"),      # block 2^13
        ((2, 16, 768, 32768, 64, 0), N.LWL_ERR_INVALID, "layers must be 1, 2, or 3"),
        ((2, 1 << 20, 1024, 32768, 64, 3), N.LWL_ERR_UNSUPPORTED, "2^30"),
        ((2, 16, 768, 32768, 1 << 20, 3), N.LWL_ERR_UNSUPPORTED, "2^29"),   # float32 partials past 2 GiB
    ],
)
def test_linear_backward_latent_validation(args, code, msg):
    lib = N.lib()
    assert lib.lwl_bfht_check_linear_backward_latent(*args) == code
    if msg:
        assert msg in lib.lwl_last_error().decode()


def test_linear_backward_latent_workspace_size():
    # 72 tiles of 256 x 128 -> 3 token splits of float32 grad_weight partials (3 x 768 x 3072),
    # their bf16 sum over 72 whole blocks, then the backward's 72 block rows (float32-sized)
    lib = N.lib()
    assert lib.lwl_bfht_linear_backward_latent_workspace_size(4096, 768, 3072, 32768) == (
        3 * 768 * 3072 * 4 + 72 * 32768 * 2 + 72 * 32768 * 4)
    # 2 x 1 tiles, 4 token steps -> 4 splits of 77 * 300 floats (padded to 64), 1 block
    assert lib.lwl_bfht_linear_backward_latent_workspace_size(200, 77, 300, 32768) == (
        4 * ceil_div(77 * 300, 64) * 64 * 4 + 32768 * 2 + 32768 * 4)


def weight_job(n, size, ld=0, wd=0, layers=2, ptr=0x10000, **kw):
    j = N.WeightJob()
    j.latent = j.weight = j.grad_weight = j.grad_latent = ptr
    j.latent_size, j.size, j.layers, j.seed = n, size, layers, 1
    j.latent_dtype, j.weight_dtype, j.weight_scale = ld, wd, 1.0
    for k, v in kw.items():
        setattr(j, k, v)
    return j


def check_jobs(jobs, forward=1):
    arr = (N.WeightJob * max(1, len(jobs)))(*jobs)
    rc = N.lib().lwl_bfht_check_weight_jobs(arr, len(jobs), forward)
    return rc, N.lib().lwl_last_error().decode()


def test_weight_job_struct_matches_header():
    # ctypes mirror of lwl_bfht_weight_job: 4 pointers, 4 int64, 2 int32, double, int32
    assert N.WeightJob.weight_scale.offset == 72 and N.WeightJob.accumulate.offset == 80
    assert ctypes_sizeof(N.WeightJob) == 88


def ctypes_sizeof(t):
    import ctypes

    return ctypes.sizeof(t)


@pytest.mark.parametrize(
    "jobs, forward, code, msg",
    [
        ([], 1, N.LWL_OK, ""),
        ([weight_job(23593, 768 * 3072, ld=0, wd=2)], 1, N.LWL_OK, ""),
        ([weight_job(32768, 1 << 20, ld=2, wd=2)], 0, N.LWL_OK, ""),
        ([weight_job(32769, 1 << 20)], 1, N.LWL_ERR_UNSUPPORTED, "blocks up to 2^15"),
        # bf16 latent of block 2^15 (matrix cores) cached as float32: per-module path
        ([weight_job(32768, 1 << 20, ld=2, wd=0)], 1, N.LWL_ERR_UNSUPPORTED, "need a bfloat16 weight"),
        # ... unless the source is not 16-byte aligned (the per-module call then uses the block kernel)
        ([weight_job(32768, 1 << 20, ld=2, wd=0, ptr=0x10002)], 1, N.LWL_OK, ""),
        ([weight_job(100, 1000, layers=4)], 1, N.LWL_ERR_INVALID, "layers must be 1, 2, or 3"),
        ([weight_job(100, 1000, wd=7)], 1, N.LWL_ERR_UNSUPPORTED, "weight dtype code 7"),
        ([weight_job(100, 0)], 1, N.LWL_ERR_INVALID, "size must be positive"),
        ([weight_job(100, 1000, weight=None)], 1, N.LWL_ERR_INVALID, "latent and weight must be non-null"),
        ([weight_job(100, 1000, grad_latent=None)], 0, N.LWL_ERR_INVALID, "grad_weight and grad_latent"),
        # destinations: weights [0x10000, +4000) and [0x10f00, ...) overlap
        ([weight_job(100, 1000), weight_job(100, 1000, weight=0x10f00)], 1, N.LWL_ERR_INVALID,
         "jobs 0 and 1 write overlapping memory"),
        ([weight_job(100, 1000), weight_job(100, 1000, weight=0x10000 + 4000)], 1, N.LWL_OK, ""),
        # flush destinations are the latent gradients (100 floats)
        ([weight_job(100, 1000), weight_job(100, 1000, grad_latent=0x10000 + 396)], 0, N.LWL_ERR_INVALID,
         "overlapping"),
    ],
)
def test_weight_job_validation(jobs, forward, code, msg):
    rc, err = check_jobs(jobs, forward)
    assert rc == code, err
    assert msg in err


def test_flush_workspace_size():
    jobs = [weight_job(23593, 768 * 3072, ptr=1 << 20), weight_job(5898, 768 * 768, ptr=2 << 20),
            weight_job(3, 7, ptr=3 << 20)]
    arr = (N.WeightJob * 3)(*jobs)
    got = N.lib().lwl_bfht_flush_weight_grads_workspace_size(arr, 3)

    def al(v):
        return (v + 255) // 256 * 256

    # one float32 partial row per block, rows 128-byte aligned (n rounded up to 32), per job 256-byte aligned
    assert got == al(72 * 23616 * 4) + al(72 * 5920 * 4) + al(2 * 32 * 4)
    bad = (N.WeightJob * 1)(weight_job(40000, 100))
    assert N.lib().lwl_bfht_flush_weight_grads_workspace_size(bad, 1) == 0


def test_batched_linears_fail_loudly_on_cpu():
    from latent_weight_lab_amd import BlockFHTLinear, block_fht_grouped_input_linear, block_fht_headwise_linear

    heads = [BlockFHTLinear(8, 4, latent_dim=8, layers=1, seed=i) for i in range(2)]
    with pytest.raises(RuntimeError, match="GPU only"):
        block_fht_headwise_linear(torch.zeros(3, 8), heads)
    with pytest.raises(RuntimeError, match="GPU only"):
        block_fht_grouped_input_linear(torch.zeros(3, 16), heads)


@pytest.mark.parametrize(
    "args, code, msg",
    [
        ((0, 10, 768), N.LWL_OK, ""),
        ((2, 0, 32768), N.LWL_OK, ""),
        ((0, 10, 32769), N.LWL_ERR_UNSUPPORTED, "up to 32768 features"),
        ((0, -1, 8), N.LWL_ERR_INVALID, "rows must be non-negative"),
        ((0, 1, 0), N.LWL_ERR_INVALID, "features must be positive"),
        ((5, 1, 8), N.LWL_ERR_UNSUPPORTED, "dtype code 5"),
    ],
)
def test_fht_mix_validation(args, code, msg):
    rc = N.lib().lwl_fht_check_mix(*args)
    assert rc == code
    assert msg in N.lib().lwl_last_error().decode()


def linear_job(tokens, in_f, out_f, n, layers=3, out=0x100000, inp=0x10000, lat=0x20000):
    j = N.LinearJob()
    j.input, j.latent, j.out = inp, lat, out
    j.tokens, j.in_features, j.latent_size, j.out_features = tokens, in_f, n, out_f
    j.layers, j.seed, j.weight_scale = layers, 1, 1.0
    return j


def test_linear_jobs_validation():
    lib = N.lib()
    ok = [linear_job(1, 768, 2304, 32768, out=0x100000), linear_job(1, 3072, 768, 32768, out=0x200000)]
    arr = (N.LinearJob * 2)(*ok)
    assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_OK
    # overlapping outputs (the second starts inside the first's 2304 bf16 values)
    arr = (N.LinearJob * 2)(linear_job(1, 768, 2304, 32768, out=0x100000), linear_job(1, 768, 768, 32768, out=0x100010))
    assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_ERR_INVALID
    assert "overlapping" in lib.lwl_last_error().decode()
    # an output over another job's input, latent, base or bias (jobs do not run in job order)
    for kw, what in ((dict(inp=0x100000), "input"), (dict(lat=0x100100), "latent")):
        arr = (N.LinearJob * 2)(linear_job(1, 768, 2304, 32768, out=0x100000),
                                linear_job(1, 768, 768, 32768, out=0x200000, **kw))
        assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_ERR_INVALID
        assert f"job 0's output overlaps job 1's {what}" in lib.lwl_last_error().decode()
    for field, ptr, what in (("base", 0x200400, "base"), ("bias", 0x2005fe, "bias")):
        epi = N.LinearEpilogue()
        setattr(epi, field, ptr)
        j1 = linear_job(1, 768, 2304, 32768, out=0x100000)
        j1.epilogue = ctypes.pointer(epi)
        arr = (N.LinearJob * 2)(j1, linear_job(1, 768, 768, 32768, out=0x200000))
        assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_ERR_INVALID
        assert f"job 1's output overlaps job 0's {what}" in lib.lwl_last_error().decode()
    # a job's own base may be its output (in place, as its single call allows)
    epi = N.LinearEpilogue()
    epi.base = 0x100000
    j0 = linear_job(1, 768, 2304, 32768, out=0x100000)
    j0.epilogue = ctypes.pointer(epi)
    arr = (N.LinearJob * 2)(j0, linear_job(1, 768, 768, 32768, out=0x200000))
    assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_OK
    # a job outside every fused kernel names its index
    arr = (N.LinearJob * 2)(linear_job(1, 768, 2304, 32768), linear_job(1, 768, 64, 16384, out=0x200000))
    assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_ERR_UNSUPPORTED
    assert lib.lwl_last_error().decode().startswith("job 1:")
    # workspace: the grouped jobs' (fewer than 256 tokens) side by side, plus the largest of the jobs
    # that run as single calls one after another (300 and 400 tokens: the tiled-x path)
    one = lib.lwl_bfht_linear_forward_workspace_size(300, 1024, 300, 32768)
    big = lib.lwl_bfht_linear_forward_workspace_size(400, 1024, 300, 32768)
    two = lib.lwl_bfht_linear_forward_workspace_size(17, 768, 768, 32768)
    three = lib.lwl_bfht_linear_forward_workspace_size(5, 3072, 768, 32768)
    arr = (N.LinearJob * 4)(linear_job(300, 1024, 300, 32768), linear_job(17, 768, 768, 32768, out=0x9000000),
                            linear_job(400, 1024, 300, 32768, out=0x20000000),
                            linear_job(5, 3072, 768, 32768, out=0x30000000))
    assert one < big
    assert lib.lwl_bfht_linear_forward_grouped_workspace_size(2, arr, 4) == two + three + big


def test_linear_workspace_three_block_tiles():
    # rows of 3072 from 2048 tokens on (tiled x): tiles of three blocks = 32 whole rows, whose
    # k-major table (96 k steps x (4 x 32 + 1) 16-byte slots) exceeds the 160 KiB LDS; the LDS
    # holds the first 76 steps (79 fit, in whole rounds of 4) and every work item (24 row tiles x
    # 256 // 24 = 10 token splits) keeps the other 20 steps' W tiles, 2 row tiles x 1 KiB each,
    # and a staging area for one block's generated chunks (8 x 16 bytes per thread of 512)
    lib = N.lib()
    assert (160 * 1024 // 16) // (4 * 32 + 1) // 4 * 4 == 76
    overflow = 24 * 10 * ((96 - 76) * 2 * 1024 + 8 * 512 * 16)
    tiled_x = (4096 // 16) * 96 * 1024
    assert lib.lwl_bfht_linear_forward_workspace_size(4096, 3072, 768, 32768) == overflow + tiled_x
    # below 2048 tokens: two-block tiles (36 for 72 blocks), whose straddling rows keep two
    # float32 partial sums per token, 256-byte aligned
    partial = (36 * 2 * 2047 * 4 + 255) // 256 * 256
    assert lib.lwl_bfht_linear_forward_workspace_size(2047, 3072, 768, 32768) == partial + 128 * 96 * 1024


def test_linear_job_and_epilogue_structs_match_header():
    # lwl_bfht_linear_job: 3 pointers, 6 int64, double, epilogue pointer;
    # lwl_bfht_linear_epilogue: 3 pointers, double
    assert N.LinearJob.weight_scale.offset == 72 and N.LinearJob.epilogue.offset == 80
    assert ctypes_sizeof(N.LinearJob) == 88
    assert N.LinearEpilogue.row_sum_scale.offset == 24 and ctypes_sizeof(N.LinearEpilogue) == 32


def test_linear_epilogue_workspace_size():
    import ctypes

    lib = N.lib()
    ep = N.LinearEpilogue()
    ep.bias, ep.base = 0x1000, 0x2000
    # no epilogue, or one without a row-sum term: the plain call's workspace (the dtype-less
    # query gives the largest over dtypes: bfloat16 at block 2^15, float32 below)
    for dtype, shape in [(2, (4096, 768, 3072, 32768)), (2, (300, 1000, 450, 32768)), (0, (300, 1024, 4096, 16384))]:
        plain = lib.lwl_bfht_linear_forward_workspace_size(*shape)
        assert lib.lwl_bfht_linear_forward_ex_workspace_size(dtype, *shape, None) == plain
        assert lib.lwl_bfht_linear_forward_ex_workspace_size(dtype, *shape, ctypes.byref(ep)) == plain
    # a row-sum term adds the float32 row sums of x, 256-byte aligned, after it
    ep.row_sum_coef = 0x3000
    plain = lib.lwl_bfht_linear_forward_workspace_size(4096, 768, 3072, 32768)
    assert lib.lwl_bfht_linear_forward_ex_workspace_size(2, 4096, 768, 3072, 32768, ctypes.byref(ep)) == plain + 4096 * 4
    assert lib.lwl_bfht_linear_forward_ex_workspace_size(0, 37, 64, 200, 4096, ctypes.byref(ep)) == 256
    # the dtype matters for the domain: float32 at block 2^15 takes no fused kernel
    assert lib.lwl_bfht_linear_forward_ex_workspace_size(0, 4096, 768, 3072, 32768, None) == 0
    assert lib.lwl_bfht_check_linear_forward(0, 4096, 768, 32768, 3072, 3) == N.LWL_ERR_UNSUPPORTED
    # grouped: a bias-only job stays grouped (its partial rows in the shared region); a job with a
    # row-sum term runs as a single launch with its row sums after its own workspace
    j1 = linear_job(17, 768, 768, 32768, out=0x9000000)
    j2 = linear_job(5, 3072, 768, 32768, out=0x30000000)
    bias_ep = N.LinearEpilogue()
    bias_ep.bias = 0x1000
    j1.epilogue = ctypes.pointer(bias_ep)
    j2.epilogue = ctypes.pointer(ep)
    two = lib.lwl_bfht_linear_forward_workspace_size(17, 768, 768, 32768)
    three = lib.lwl_bfht_linear_forward_workspace_size(5, 3072, 768, 32768)
    arr = (N.LinearJob * 2)(j1, j2)
    assert lib.lwl_bfht_check_linear_jobs(2, arr, 2) == N.LWL_OK
    assert lib.lwl_bfht_linear_forward_grouped_workspace_size(2, arr, 2) == two + three + 256
