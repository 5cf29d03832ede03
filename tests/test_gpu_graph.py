"""The C-ABI entry points under HIP graph capture: each call is captured once into a graph,
which is replayed three times; before every replay the outputs are poisoned with NaN by an
eager fill kernel and other eager library calls run (reusing the library's scratch and torch's
memory), and after it every output equals the eager call's bit for bit (the kernels are
deterministic).  The library records no memset, copy, allocation or synchronization, so
captured calls replay the same launches with the same arguments.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import gpu_available
from latent_weight_lab_amd import _native as N
from latent_weight_lab_amd import ops

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def disturb():
    """Eager library work between replays: other shapes through the same kernels."""
    g = torch.Generator(device="cuda").manual_seed(99)
    lat = torch.randn(32768, device="cuda", generator=g).to(torch.bfloat16)
    ops.forward(lat, 32768 * 8, 3, 1, 0, 32768 * 8)
    ops.backward(torch.randn(5000, device="cuda", generator=g), 3000, torch.float32, 5000, 2, 4, 0, 5000)
    x = torch.randn(20, 768, device="cuda", generator=g).to(torch.bfloat16)
    ops.linear_forward(x, lat, 768, 3, 5, 1.0)
    # the no-allocation backward on another shape: replays then run over its reused scratch array
    gr = torch.randn(108_618, device="cuda", generator=g)
    gl = torch.empty(1024, device="cuda")
    lib = N.lib()
    rc = lib.lwl_bfht_backward_noalloc(gr.data_ptr(), N.dtype_code(torch.float32), 1024, 108_618, 3, 123, 0,
                                       108_618, gl.data_ptr(), ctypes.c_void_p(N.stream_ptr(gr.device)))
    assert rc == N.LWL_OK, lib.lwl_last_error().decode()


def check_graph(fn):
    """Eager outputs of fn(), then fn captured and replayed 3 times against them."""
    want = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up outside the capture, as torch requires
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        disturb()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), (rep, i)


def test_graph_forward_backward():
    g = torch.Generator(device="cuda").manual_seed(1)
    lat16 = torch.randn(32768, device="cuda", generator=g).to(torch.bfloat16)
    lat32 = torch.randn(1 << 20, device="cuda", generator=g)
    grad16 = torch.randn(64 * 32768, device="cuda", generator=g).to(torch.bfloat16)
    grad32 = torch.randn(1 << 22, device="cuda", generator=g)

    def fn():
        return [ops.forward(lat16, 64 * 32768, 3, 7, 0, 64 * 32768),                 # matrix cores, whole blocks
                ops.forward(lat16, 64 * 32768, 3, 7, 12345, 1_012_345),              # slice
                ops.backward(grad16, 32768, torch.bfloat16, 64 * 32768, 3, 7, 0, 64 * 32768),
                ops.forward(lat32, 1 << 22, 3, 99, 0, 1 << 22),                      # block 2^20: tile passes
                ops.backward(grad32, 1 << 20, torch.float32, 1 << 22, 3, 99, 0, 1 << 22)]

    check_graph(fn)


def test_graph_fused_linear():
    g = torch.Generator(device="cuda").manual_seed(2)
    lat = torch.randn(32768, device="cuda", generator=g).to(torch.bfloat16)
    x64 = torch.randn(64, 768, device="cuda", generator=g).to(torch.bfloat16)
    x300 = torch.randn(300, 768, device="cuda", generator=g).to(torch.bfloat16)
    bias = torch.randn(3072, device="cuda", generator=g).to(torch.bfloat16)
    coef = torch.tensor([0.01], device="cuda")
    lat_ref = torch.randn(16384, device="cuda", generator=g).to(torch.float16)
    xr = torch.randn(300, 1024, device="cuda", generator=g).to(torch.float16)
    xr5 = torch.randn(5, 1024, device="cuda", generator=g).to(torch.float16)
    x3k = torch.randn(3100, 3072, device="cuda", generator=g).to(torch.bfloat16)
    bias768 = torch.randn(768, device="cuda", generator=g).to(torch.bfloat16)

    def fn():
        return [ops.linear_forward(x64, lat, 3072, 3, 3, 1.0),
                ops.linear_forward(x300, lat, 3072, 3, 3, 1.0, bias=bias, row_sum_coef=coef),  # tiled x, epilogue
                ops.linear_forward(xr, lat_ref, 4096, 2, 123, 0.5),   # reference domain, matrix cores
                ops.linear_forward(xr5, lat_ref, 4096, 2, 123, 0.5),  # reference domain, VALU
                # three-block tiles: overflow W tiles and a staged block round-trip through the workspace
                ops.linear_forward(x3k, lat, 700, 3, 3, 0.5, bias=bias768[:700])]

    check_graph(fn)


def test_graph_grouped_linear_and_weight_cache():
    g = torch.Generator(device="cuda").manual_seed(3)
    lats = [torch.randn(32768, device="cuda", generator=g).to(torch.bfloat16) for _ in range(4)]
    shapes = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
    xs = {i: torch.randn(9, i, device="cuda", generator=g).to(torch.bfloat16) for i in (768, 3072)}
    biases = [torch.randn(o, device="cuda", generator=g).to(torch.bfloat16) for _, o in shapes]
    specs = [(xs[i], lat, o, 3, 100 + k, 1.0, {"bias": b}) for k, ((i, o), lat, b) in enumerate(zip(shapes, lats, biases))]
    lat32 = [torch.randn(n, device="cuda", generator=g) for n in (5898, 492, 23593)]
    wspecs = [(lat, size, 2, 1000 + k, 0.5, torch.bfloat16)
              for k, (lat, size) in enumerate(zip(lat32, (768 * 768, 768 * 64, 768 * 3072)))]
    gws = [torch.randn(size, device="cuda", generator=g).to(torch.bfloat16) for _, size, *_ in wspecs]
    fspecs = [(lat, gw, size, 2, 1000 + k, 0.5, None) for k, ((lat, size, *_), gw) in enumerate(zip(wspecs, gws))]

    def fn():
        return (ops.linear_forward_grouped(specs) + ops.materialize_weights(wspecs)
                + ops.flush_weight_grads(fspecs))

    check_graph(fn)


def test_graph_noalloc_backward_and_mix():
    g = torch.Generator(device="cuda").manual_seed(4)
    grad = torch.randn(8 * 32768, device="cuda", generator=g)
    x = torch.randn(512, 768, device="cuda", generator=g).to(torch.bfloat16)
    signs = (torch.randint(0, 2, (1024,), device="cuda", generator=g) * 2 - 1).float()
    lib = N.lib()

    def fn():
        gl = torch.empty(32768, device="cuda")
        rc = lib.lwl_bfht_backward_noalloc(grad.data_ptr(), N.dtype_code(torch.float32), 32768, 8 * 32768, 3, 7,
                                           0, 8 * 32768, gl.data_ptr(), ctypes.c_void_p(N.stream_ptr(grad.device)))
        assert rc == N.LWL_OK, lib.lwl_last_error().decode()
        return [gl, ops.fht_mix(x, signs)]

    check_graph(fn)


def test_graph_linear_latent_gradient():
    g = torch.Generator(device="cuda").manual_seed(5)
    lat = torch.randn(32768, device="cuda", generator=g).to(torch.bfloat16)
    x = torch.randn(300, 768, device="cuda", generator=g).to(torch.bfloat16)
    gr = torch.randn(300, 3072, device="cuda", generator=g).to(torch.bfloat16)
    x77 = torch.randn(50, 77, device="cuda", generator=g).to(torch.bfloat16)
    g77 = torch.randn(50, 300, device="cuda", generator=g).to(torch.bfloat16)

    def fn():
        return [ops.linear_backward_latent(gr, x, lat, 3072, 3, 3, 0.5),      # split-K over 5 token steps
                ops.linear_backward_latent(g77, x77, lat, 300, 2, 13, 1.0)]   # element loads

    check_graph(fn)
