"""The no-allocation backward ``lwl_bfht_backward_noalloc`` (scratch in a file-scope device
array instead of a workspace) against ``lwl_bfht_backward`` with a workspace, through the C ABI:
bit-identical gradients (same kernels, same fixed-order block sum), on calls in a row where each
later call is smaller than the one before (the scratch then still holds the earlier call's
partial rows, which the kernels must fully overwrite).  The refusal of a call whose scratch
exceeds the array happens on the host before any HIP call and is tested on the CPU
(tests/test_abi_cpu.py)."""
from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import _native as N
from latent_weight_lab_amd import ops

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def noalloc_backward(grad, n, dtype, size, layers, seed, start, stop):
    out = torch.empty(n, dtype=dtype, device=grad.device)
    lib = N.lib()
    rc = lib.lwl_bfht_backward_noalloc(grad.data_ptr(), N.dtype_code(dtype), n, size, layers, seed, start, stop,
                                       out.data_ptr(), N.stream_ptr(grad.device))
    N.check(rc)
    return out


def with_workspace(grad, n, dtype, size, layers, seed, start, stop):
    return ops.backward(grad, n, dtype, size, layers, seed, start, stop)


# each call smaller than the one before: (latent size, size, layers, seed, start, stop, dtype)
CALLS = [
    (32768, 8_388_608, 3, 7, 0, 8_388_608, torch.float32),      # config 2 fp32: 256 rows, all 32 MiB
    (32768, 8_388_608, 3, 7, 12_345, 1_012_345, torch.bfloat16),  # config 2 slice, matrix cores: 31 rows
    (1024, 108_618, 3, 123, 0, 108_618, torch.float32),         # config 1: 107 rows of 1024
    (1000, 5_000, 2, 9, 17, 3_000, torch.float16),              # 3 rows
]


def test_noalloc_backward_matches_workspace_backward():
    print(f"no-alloc scratch array: {32 << 20} bytes", flush=True)
    for n, size, layers, seed, start, stop, dtype in CALLS:
        print(f"case n={n} size={size} layers={layers} seed={seed} [{start},{stop}) {dtype}", flush=True)
        need = N.lib().lwl_bfht_backward_workspace_size(n, size, start, stop)
        assert 0 < need <= 32 << 20
        g = torch.randn(stop - start, generator=torch.Generator().manual_seed(n + start)).to(dtype).cuda()
        got = noalloc_backward(g, n, dtype, size, layers, seed, start, stop)
        want = with_workspace(g, n, dtype, size, layers, seed, start, stop)
        torch.cuda.synchronize()
        assert got.dtype == want.dtype and got.shape == want.shape
        assert torch.equal(got, want), (n, size, start, stop, dtype)


def test_noalloc_backward_twice_in_a_row_same_stream_state():
    # the first call fills the scratch; a smaller second call on the same stream must not see it
    big = torch.randn(8_388_608, generator=torch.Generator().manual_seed(1)).cuda()
    small = torch.randn(4_000, generator=torch.Generator().manual_seed(2)).cuda()
    a1 = noalloc_backward(big, 32768, torch.float32, 8_388_608, 3, 7, 0, 8_388_608)
    a2 = noalloc_backward(small, 2000, torch.float32, 4_000, 3, 7, 0, 4_000)
    b1 = with_workspace(big, 32768, torch.float32, 8_388_608, 3, 7, 0, 8_388_608)
    b2 = with_workspace(small, 2000, torch.float32, 4_000, 3, 7, 0, 4_000)
    torch.cuda.synchronize()
    assert torch.equal(a1, b1) and torch.equal(a2, b2)

