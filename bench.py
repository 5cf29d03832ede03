"""Benchmark of the BlockFHT hot path on one MI355X.

Headline (BASELINE metric, config 2): full BlockFHT generation at
block_size = 32768, layers = 3, hash seed 7, 256 blocks (8,388,608
coordinates), bfloat16 latent/output, latent ~N(0,1) from torch seed 1.  One
step = one call of the C ABI forward (``lwl_bfht_forward``) over the whole
output, inputs resident in HBM.  The K timed steps are captured into one HIP
graph and replayed once, bracketed by HIP events on the capture stream, so the
timed region measures the GPU back to back (a Python launch costs more than
the kernel).

Printed: one JSON line with the contract keys, plus
  roofline      algorithmic HBM bytes per launch / average launch duration;
  cpu_baseline  the reference's CPU fallback algorithm (op-for-op torch port,
                oracle/oracle.py) timed on this host on the same workload;
  extra         the other configs' directions and dtypes (backward, float32,
                slice, multi-pass 2^20 / 2^23, fused linear vs dense GEMM).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
BF16_MFMA_PEAK_TFLOPS = 2500.0  # dense


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-extra", action="store_true", help="headline only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--only", default="", help="comma list of extra names to run (default: all)")
    p.add_argument("--eager", action="store_true",
                   help="time the headline with eager launches instead of one graph replay (for counter runs)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 64 MiB device-to-device copy 20 times (reference kernel for the HBM byte "
                        "counters: FETCH_SIZE/WRITE_SIZE per dispatch vs 64 MiB read and written)")
    return p.parse_args()


# ---------------------------------------------------------------- helpers

class Abi:
    """Direct C-ABI calls on preallocated buffers (what a drop-in caller does)."""

    def __init__(self):
        import torch

        from latent_weight_lab_amd import _native as N

        self.torch = torch
        self.N = N
        self.lib = N.lib()

    def stream(self):
        return self.torch.cuda.current_stream().cuda_stream

    def forward(self, latent, out, size, layers, seed, start, stop, ws=None):
        N = self.N
        wp, wn = (ws.data_ptr(), ws.numel()) if ws is not None else (0, 0)
        rc = self.lib.lwl_bfht_forward(latent.data_ptr(), N.dtype_code(latent.dtype), latent.numel(), size,
                                       layers, seed, start, stop, out.data_ptr(), wp, wn, self.stream())
        N.check(rc)

    def backward(self, grad, grad_latent, size, layers, seed, start, stop, ws=None):
        N = self.N
        wp, wn = (ws.data_ptr(), ws.numel()) if ws is not None else (0, 0)
        rc = self.lib.lwl_bfht_backward(grad.data_ptr(), N.dtype_code(grad.dtype), grad_latent.numel(), size,
                                        layers, seed, start, stop, grad_latent.data_ptr(), wp, wn, self.stream())
        N.check(rc)

    def linear(self, x, latent, out, out_f, layers, seed, scale, ws=None):
        N = self.N
        tokens, in_f = x.shape
        wp, wn = (ws.data_ptr(), ws.numel()) if ws is not None else (0, 0)
        rc = self.lib.lwl_bfht_linear_forward(x.data_ptr(), latent.data_ptr(), N.dtype_code(x.dtype), tokens, in_f,
                                              latent.numel(), out_f, layers, seed, scale, out.data_ptr(), wp, wn,
                                              self.stream())
        N.check(rc)

    def linear_ws(self, tokens, in_f, out_f, n, device):
        nbytes = self.lib.lwl_bfht_linear_forward_workspace_size(tokens, in_f, out_f, n)
        return self.torch.empty(nbytes, dtype=self.torch.uint8, device=device) if nbytes else None

    def fwd_ws(self, n, size, start, stop, device):
        nbytes = self.lib.lwl_bfht_forward_workspace_size(n, size, start, stop)
        return self.torch.empty(nbytes, dtype=self.torch.uint8, device=device) if nbytes else None

    def bwd_ws(self, n, size, start, stop, device):
        nbytes = self.lib.lwl_bfht_backward_workspace_size(n, size, start, stop)
        return self.torch.empty(nbytes, dtype=self.torch.uint8, device=device) if nbytes else None

    def linear_bwd_latent(self, grad, x, latent, grad_latent, out_f, layers, seed, scale, ws):
        N = self.N
        tokens, in_f = x.shape
        rc = self.lib.lwl_bfht_linear_backward_latent(grad.data_ptr(), x.data_ptr(), N.dtype_code(x.dtype), tokens,
                                                      in_f, latent.numel(), out_f, layers, seed, float(scale),
                                                      grad_latent.data_ptr(), ws.data_ptr(), ws.numel(),
                                                      self.stream())
        N.check(rc)

    def linear_bwd_ws(self, tokens, in_f, out_f, n, device):
        nbytes = self.lib.lwl_bfht_linear_backward_latent_workspace_size(tokens, in_f, out_f, n)
        return self.torch.empty(nbytes, dtype=self.torch.uint8, device=device)


# A GPU idle until the timed region runs its first ~25 ms of work at lower
# clocks: the config-2 forward takes 9.2-9.3 us per step cold and 8.3 us after
# ~25 ms of back-to-back launches, and is cold again after 0.5 s idle.  The
# headline therefore runs its own workload for SETTLE_S first (untimed,
# reported in the JSON line), then the W warm-up steps and the K timed steps.
SETTLE_S = 0.05


def settle(torch, g, seconds: float) -> int:
    """Replays graph g (synchronizing after each replay, so the queue stays
    short) until `seconds` of wall time have passed; returns the replays."""
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        g.replay()
        torch.cuda.synchronize()
        n += 1
    return n


def time_graph(torch, fn, steps: int, warmup: int, settle_s: float = 0.0, info: dict | None = None) -> float:
    """Seconds per step: `steps` calls of fn captured in one HIP graph,
    replayed once between events recorded on the capture stream.  With
    settle_s > 0, a graph of 100 calls is replayed for that long first."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(1, warmup)):
            fn()  # eager warm-up (also settles lazily-created state)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g_warm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_warm):
        for _ in range(max(1, warmup)):
            fn()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(steps):
            fn()
    if settle_s > 0:
        g_settle = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_settle):
            for _ in range(100):
                fn()
        n = settle(torch, g_settle, settle_s)
        if info is not None:
            info["settle_s"] = settle_s
            info["settle_steps"] = 100 * n
        del g_settle
    g_warm.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / steps


def time_eager(torch, fn, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / steps


def profiled_traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, each scaled by the same
    counter on a plain copy of known size), read from the committed summary in profiles/."""
    path = ROOT / "profiles" / name
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def config2_latent(torch, dtype):
    torch.manual_seed(1)
    return torch.randn(32768, dtype=torch.float32).to(dtype)


def config1_latent(torch):
    torch.manual_seed(0)
    return torch.randn(1024, dtype=torch.float32)


# ---------------------------------------------------------------- headline

C1_N = 1024
C1_SIZE = 108_618
C2_N = 32768
C2_SIZE = 8_388_608
C2_LAYERS = 3
C2_SEED = 7


def headline(abi, steps, warmup, eager=False, info=None):
    torch = abi.torch
    dt = torch.bfloat16
    latent = config2_latent(torch, dt).cuda()
    out = torch.empty(C2_SIZE, dtype=dt, device="cuda")
    ws = abi.fwd_ws(C2_N, C2_SIZE, 0, C2_SIZE, "cuda")

    def step():
        abi.forward(latent, out, C2_SIZE, C2_LAYERS, C2_SEED, 0, C2_SIZE, ws)

    if eager:
        sec = time_eager(torch, step, steps, warmup)
    else:
        sec = time_graph(torch, step, steps, warmup, settle_s=SETTLE_S, info=info)
    return sec, out


# ---------------------------------------------------------------- extra configs

def extra_configs(abi, steps, warmup, only):
    torch = abi.torch
    res = {}

    def want(name):
        return not only or name in only

    def run(name, fn, nbytes, coords, graph=True, nsteps=None):
        if not want(name):
            return
        try:
            k = nsteps or steps
            sec = time_graph(torch, fn, k, warmup) if graph else time_eager(torch, fn, k, warmup)
            res[name] = {"ms": round(sec * 1e3, 5), "coords_per_s": coords / sec,
                         "algo_GBs": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS}
        except Exception as exc:  # noqa: BLE001 - reported, not fatal
            res[name] = {"error": f"{type(exc).__name__}: {exc}"}

    # config 1 (the reference's CPU-runnable case): n = 1024, size 108,618, layers 3, seed 123, fp32
    lat1 = config1_latent(torch).cuda()
    out1 = torch.empty(C1_SIZE, dtype=torch.float32, device="cuda")
    sl1 = torch.empty(1000, dtype=torch.float32, device="cuda")
    g1 = torch.randn(C1_SIZE, generator=torch.Generator().manual_seed(4)).cuda()
    gl1 = torch.empty(C1_N, dtype=torch.float32, device="cuda")
    bws1 = abi.bwd_ws(C1_N, C1_SIZE, 0, C1_SIZE, "cuda")
    run("c1_fwd_f32", lambda: abi.forward(lat1, out1, C1_SIZE, 3, 123, 0, C1_SIZE), C1_SIZE * 4 + C1_N * 4, C1_SIZE)
    run("c1_slice_f32", lambda: abi.forward(lat1, sl1, C1_SIZE, 3, 123, 1000, 2000), 1000 * 4 + C1_N * 4, 1000)
    run("c1_bwd_f32", lambda: abi.backward(g1, gl1, C1_SIZE, 3, 123, 0, C1_SIZE, bws1), C1_SIZE * 4 + C1_N * 4,
        C1_SIZE)
    del lat1, out1, sl1, g1, gl1, bws1

    for dt, es in ((torch.bfloat16, 2), (torch.float32, 4)):
        tag = "bf16" if dt == torch.bfloat16 else "f32"
        latent = config2_latent(torch, dt).cuda()
        out = torch.empty(C2_SIZE, dtype=dt, device="cuda")
        grad = torch.randn(C2_SIZE, generator=torch.Generator().manual_seed(5)).to(dt).cuda()
        gl = torch.empty(C2_N, dtype=dt, device="cuda")
        bws = abi.bwd_ws(C2_N, C2_SIZE, 0, C2_SIZE, "cuda")
        if tag == "f32":
            run(f"c2_fwd_{tag}", lambda: abi.forward(latent, out, C2_SIZE, 3, 7, 0, C2_SIZE),
                C2_SIZE * es + C2_N * es, C2_SIZE)
        run(f"c2_bwd_{tag}", lambda: abi.backward(grad, gl, C2_SIZE, 3, 7, 0, C2_SIZE, bws),
            C2_SIZE * es + C2_N * es, C2_SIZE)
        s0, s1 = 12_345, 1_012_345
        sl = torch.empty(s1 - s0, dtype=dt, device="cuda")
        run(f"c2_slice_{tag}", lambda: abi.forward(latent, sl, C2_SIZE, 3, 7, s0, s1),
            (s1 - s0) * es + C2_N * es, s1 - s0)
        gs = grad[s0:s1]  # the slice's gradient where it lies in the full one (2-byte offset)
        sws = abi.bwd_ws(C2_N, C2_SIZE, s0, s1, "cuda")
        run(f"c2_slice_bwd_{tag}", lambda: abi.backward(gs, gl, C2_SIZE, 3, 7, s0, s1, sws),
            (s1 - s0) * es + C2_N * es, s1 - s0)
        del latent, out, grad, gl, bws, sl, gs, sws

    # config 3: multi-pass blocks 2^20 and 2^23, size 2^26, fp32, layers 3, seed 99.  At ~0.4 ms per
    # call, at least 20 calls per timed graph: with 5 (the old floor at --steps 20) the calls read
    # 3-6 % slower on the same box than with 20
    size = 1 << 26
    for lb in (20, 23):
        name = f"c3_b2^{lb}"
        if not (want(name + "_fwd") or want(name + "_bwd")):
            continue
        B = 1 << lb
        torch.manual_seed(2)
        latent = torch.randn(B, dtype=torch.float32).cuda()
        out = torch.empty(size, dtype=torch.float32, device="cuda")
        fws = abi.fwd_ws(B, size, 0, size, "cuda")
        run(name + "_fwd", lambda: abi.forward(latent, out, size, 3, 99, 0, size, fws), size * 4 + B * 4, size,
            nsteps=max(20, steps // 10))
        del fws
        grad = torch.randn(size, generator=torch.Generator().manual_seed(3)).cuda()
        gl = torch.empty(B, dtype=torch.float32, device="cuda")
        bws = abi.bwd_ws(B, size, 0, size, "cuda")
        run(name + "_bwd", lambda: abi.backward(grad, gl, size, 3, 99, 0, size, bws), size * 4 + B * 4, size,
            nsteps=max(20, steps // 10))
        del latent, out, grad, gl, bws
        torch.cuda.empty_cache()

    # config 4: fused linear at GPT-2-small MLP shapes vs dense bf16 GEMM on the materialized weight
    if want("c4_linear"):
        from latent_weight_lab_amd import block_fht_linear_forward, block_fht_slice

        lin = {}
        for inf, outf in ((768, 3072), (3072, 768)):
            try:
                torch.manual_seed(3)
                latent = torch.randn(32768, dtype=torch.float32).to(torch.bfloat16).cuda()
                x = torch.randn(4096, inf, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
                out = torch.empty(4096, outf, dtype=torch.bfloat16, device="cuda")
                ws = abi.linear_ws(4096, inf, outf, 32768, "cuda")
                with torch.no_grad():
                    w = block_fht_slice(latent, inf * outf, 3, 3, 0, inf * outf).view(outf, inf)
                flops = 2 * 4096 * inf * outf
                fused = time_graph(torch, lambda: abi.linear(x, latent, out, outf, 3, 3, 1.0, ws), 50, 5)
                dense = time_graph(torch, lambda: torch.nn.functional.linear(x, w), 50, 5)
                with torch.no_grad():  # the other route: generate W once (one launch), then the GEMM
                    gen = time_graph(torch, lambda: block_fht_linear_forward(x, latent, outf, 3, 3, fused=False),
                                     50, 5)
                lin[f"{inf}x{outf}"] = {"fused_ms": round(fused * 1e3, 4),
                                        "dense_gemm_ms": round(dense * 1e3, 4),
                                        "fused_over_dense": fused / dense,
                                        "fused_tokens_per_s": 4096 / fused,
                                        "fused_TFLOPs": flops / fused / 1e12,
                                        "dense_TFLOPs": flops / dense / 1e12,
                                        "generate_then_gemm_ms": round(gen * 1e3, 4),
                                        "generate_then_gemm_over_dense": gen / dense}
                del latent, x, out, ws, w
            except Exception as exc:  # noqa: BLE001
                lin[f"{inf}x{outf}"] = {"error": f"{type(exc).__name__}: {exc}"}
        res["c4_linear"] = lin

    # the reference extension's own fused-linear domain (block <= 2^14, block % in == 0): its profiling
    # case (scripts/profile_fused_once.py: 1024 -> 4096, float16, latent 16384, layers 2, scale 0.5) at one
    # token and at 4096, fused (W generated into LDS in float32, never stored) vs a dense float16 GEMM on
    # the materialized weight
    if want("c4_ref_domain"):
        from latent_weight_lab_amd import block_fht_slice

        rows = {}
        for dt, tag in ((torch.float16, "f16"), (torch.float32, "f32")):
            for tokens in (1, 4096):
                try:
                    torch.manual_seed(0)
                    latent = torch.randn(16384).to(dt).cuda()
                    x = torch.randn(tokens, 1024, generator=torch.Generator().manual_seed(1)).to(dt).cuda()
                    out = torch.empty(tokens, 4096, dtype=dt, device="cuda")
                    ws = abi.linear_ws(tokens, 1024, 4096, 16384, "cuda")
                    with torch.no_grad():
                        w = block_fht_slice(latent, 1024 * 4096, 2, 123, 0, 1024 * 4096).view(4096, 1024) * 0.5
                    fused = time_graph(torch, lambda: abi.linear(x, latent, out, 4096, 2, 123, 0.5, ws), 20, 3)
                    dense = time_graph(torch, lambda: torch.nn.functional.linear(x, w), 20, 3)
                    rows[f"{tag}_tokens_{tokens}"] = {"fused_ms": round(fused * 1e3, 4), "dense_gemm_ms": round(dense * 1e3, 4),
                                                      "fused_over_dense": fused / dense,
                                                      "fused_TFLOPs": 2 * tokens * 1024 * 4096 / fused / 1e12}
                    del latent, x, out, ws, w
                except Exception as exc:  # noqa: BLE001
                    rows[f"{tag}_tokens_{tokens}"] = {"error": f"{type(exc).__name__}: {exc}"}
        res["c4_ref_domain"] = rows

    # config 4 training step, latent gradient: one lwl_bfht_linear_backward_latent call (split-K
    # matrix-core g^T x into float32 partials, their sum, the generator backward) vs the reference's
    # composition, grad_weight = g^T x on hipBLASLt followed by the generator backward
    if want("c4_linear_bwd"):
        lin = {}
        for inf, outf in ((768, 3072), (3072, 768)):
            try:
                torch.manual_seed(3)
                latent = torch.randn(32768, dtype=torch.float32).to(torch.bfloat16).cuda()
                x = torch.randn(4096, inf, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
                g = torch.randn(4096, outf, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
                gl = torch.empty(32768, dtype=torch.bfloat16, device="cuda")
                gl2 = torch.empty(32768, dtype=torch.bfloat16, device="cuda")
                ws = abi.linear_bwd_ws(4096, inf, outf, 32768, "cuda")
                size = inf * outf
                bws = abi.bwd_ws(32768, size, 0, size, "cuda")
                gw = torch.empty(outf, inf, dtype=torch.bfloat16, device="cuda")

                def unfused():
                    torch.matmul(g.t(), x, out=gw)
                    abi.backward(gw.view(-1), gl2, size, 3, 3, 0, size, bws)

                fused = time_graph(torch, lambda: abi.linear_bwd_latent(g, x, latent, gl, outf, 3, 3, 1.0, ws),
                                   20, 3)
                base = time_graph(torch, unfused, 20, 3)
                lin[f"{inf}x{outf}"] = {"fused_ms": round(fused * 1e3, 4), "unfused_ms": round(base * 1e3, 4),
                                        "fused_over_unfused": fused / base,
                                        "rel_l2_vs_unfused": float((gl.float() - gl2.float()).norm()
                                                                   / gl2.float().norm())}
                del latent, x, g, gl, gl2, ws, bws, gw
            except Exception as exc:  # noqa: BLE001
                lin[f"{inf}x{outf}"] = {"error": f"{type(exc).__name__}: {exc}"}
        res["c4_linear_bwd"] = lin

    # weight cache of the nanoGPT GPT-2-small recipe (examples/nanogpt: 48 matrices, latent ratio 0.01,
    # 2 layers, seeds 1000+i, float32 latents, bf16 cache): grouped prepare / flush (one C-ABI call each)
    # vs the per-module loop (generate, scale, cast; cast, backward, scale, accumulate per module)
    if want("c6_cache"):
        try:
            res["c6_cache"] = cache_bench(abi, torch)
        except Exception as exc:  # noqa: BLE001
            res["c6_cache"] = {"error": f"{type(exc).__name__}: {exc}"}

    # many small generators (nanoGPT HeadwiseLinear / GroupedInputLinear): one training step (forward +
    # backward) of all heads batched into one grouped generation vs head by head
    if want("c7_heads"):
        try:
            res["c7_heads"] = heads_bench(torch)
        except Exception as exc:  # noqa: BLE001
            res["c7_heads"] = {"error": f"{type(exc).__name__}: {exc}"}

    # signed activation FHT (nanoGPT FixedFHTMix) on 8192 bf16 rows: one launch vs the reference's
    # torch loop (pad, sign, log2(P) reshape/clone butterfly stages, scale, sign, slice) on this GPU
    if want("c8_mix"):
        try:
            res["c8_mix"] = mix_bench(torch)
        except Exception as exc:  # noqa: BLE001
            res["c8_mix"] = {"error": f"{type(exc).__name__}: {exc}"}

    # forward_fused's tail (bias, modulation row-sum term, residual base) in the fused kernels'
    # stores (lwl_bfht_linear_forward_ex) vs the reference's sequence of torch ops after the
    # fused linear (block_fht.py:493-500), config-4 shapes
    if want("c4_epilogue"):
        try:
            res["c4_epilogue"] = epilogue_bench(torch)
        except Exception as exc:  # noqa: BLE001
            res["c4_epilogue"] = {"error": f"{type(exc).__name__}: {exc}"}

    # config 5: 12-layer GPT-2-small linear stack (qkv, proj, fc, fc-proj per layer = 48 matrices,
    # latents of 32768 bf16, seeds 100+i), forward only, fused vs dense on materialized weights
    if want("c5_stack"):
        res["c5_stack"] = stack_bench(abi, torch)

    # the reference's own published shapes (context beside docs/block_fht_notes.md:34-39,81-85,
    # RTX 4080 prototype numbers; not targets): its block-size sweep and its stacked decode
    for name, fn in (("ref_sweep", ref_sweep_bench), ("ref_stack", ref_stack_bench)):
        if want(name):
            try:
                res[name] = fn(torch)
            except Exception as exc:  # noqa: BLE001
                res[name] = {"error": f"{type(exc).__name__}: {exc}"}
    return res


def ref_sweep_bench(torch, iters: int = 10):
    """benchmarks/bench_block_fht.py:26-49 on this GPU: for block 2^5 .. 2^23, BlockFHT of a
    float32 latent of one block, size = block, layers 1, seed = the power; forward, and forward +
    backward of mean(y^2), each timed the reference's way (wall clock, a device sync per
    iteration, 10 iterations after one warm-up slice backward; here also one untimed iteration of
    each loop first, so that no one-time first-call cost lands in its mean).  Also the device time
    of the forward in graph replay (no host or sync latency)."""
    from latent_weight_lab_amd import BlockFHT

    rows = {}
    for power in range(5, 24):
        block = 1 << power
        torch.manual_seed(power)
        m = BlockFHT(block, size=block, layers=1, seed=power).cuda()
        m.latent.data = m.latent.data.float()
        m.slice(0, min(block, 1024)).sum().backward()
        m.latent.grad = None
        torch.cuda.synchronize()

        def fwd():
            m()

        def fwd_bwd():
            m.latent.grad = None
            m().square().mean().backward()

        def wall_ms(fn):
            fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(iters):
                fn()
                torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / iters

        fwd_ms, fb_ms = wall_ms(fwd), wall_ms(fwd_bwd)
        with torch.no_grad():
            dev_ms = time_graph(torch, lambda: m(), 20, 3) * 1e3
        rows[f"2^{power}"] = {"forward_ms": round(fwd_ms, 4), "forward_backward_ms": round(fb_ms, 4),
                              "forward_device_ms": round(dev_ms, 5)}
        del m
    return {"method": "reference bench_block_fht.py (wall clock, sync per iteration, 10 iterations), fp32, "
                      "layers 1, size = block", "rows": rows}


def ref_stack_bench(torch, iters: int = 20):
    """benchmarks/bench_fused_linear_stack.py:15-84 on this GPU: tokens 1, 1024 -> 4096, one float32
    latent of 16384 shared by every matrix, layers 2, seeds 1000 + i; 1 / 4 / 16 / 64 matrices
    through the fused linear ("fused_shared_latent") against F.linear on resident materialized
    weights ("resident_dense"), each iteration ending in the reference's reduction of the
    outputs, timed its way (wall clock over 20 iterations after 3 warm-ups, peak MiB from
    max_memory_allocated after a reset).  The reference runs each mode in a process of its own;
    here the fused mode runs before the weights exist and both peaks leave out what the earlier
    bench rows still hold."""
    import torch.nn.functional as F

    from latent_weight_lab_amd import block_fht_linear_forward, block_fht_slice

    tokens, fin, fout, ld, layers = 1, 1024, 4096, 16384, 2
    torch.cuda.synchronize()
    outside = torch.cuda.memory_allocated()  # what earlier rows still hold
    torch.manual_seed(123)
    x = torch.randn(tokens, fin, device="cuda")
    latent = torch.randn(ld, device="cuda")

    def bench(weights, matrices, n):
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(n):
            outs = []
            for i in range(len(weights) if weights is not None else matrices):
                if weights is None:
                    outs.append(block_fht_linear_forward(x, latent, fout, layers, 1000 + i))
                else:
                    outs.append(F.linear(x, weights[i]))
            y = torch.stack([o.float().mean() for o in outs]).sum()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / n
        peak = (torch.cuda.max_memory_allocated() - outside) / 2**20
        float(y)
        return ms, peak

    rows = {}
    with torch.no_grad():
        for matrices in (1, 4, 16, 64):
            size = fin * fout
            for _ in range(3):
                bench(None, matrices, 1)
            f_ms, f_peak = bench(None, matrices, iters)
            weights = [block_fht_slice(latent, size, layers, 1000 + i, 0, size).view(fout, fin).clone()
                       for i in range(matrices)]
            torch.cuda.synchronize()
            for _ in range(3):
                bench(weights, matrices, 1)
            d_ms, d_peak = bench(weights, matrices, iters)
            rows[f"matrices_{matrices}"] = {"fused_ms": round(f_ms, 4), "fused_peak_MiB": round(f_peak, 1),
                                            "resident_dense_ms": round(d_ms, 4),
                                            "resident_dense_peak_MiB": round(d_peak, 1),
                                            "fused_over_dense": f_ms / d_ms}
            del weights
            torch.cuda.empty_cache()
    return {"method": "reference bench_fused_linear_stack.py (wall clock, 20 iterations), fp32, tokens 1, "
                      "1024 -> 4096, shared latent 16384, layers 2", "rows": rows}


GPT2_SHAPES = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]


def stack_bench(abi, torch):
    from latent_weight_lab_amd import block_fht_linear_forward, block_fht_slice

    mats = []
    for layer in range(12):
        for j, (inf, outf) in enumerate(GPT2_SHAPES):
            i = 4 * layer + j
            torch.manual_seed(100 + i)
            mats.append((inf, outf, torch.randn(32768).to(torch.bfloat16).cuda(), 100 + i))
    torch.cuda.synchronize()
    from latent_weight_lab_amd import ops as lwl_ops

    out = {}
    for tokens in (1, 16, 64, 8 * 1024):
        row = {}
        try:
            xs = {inf: torch.randn(tokens, inf, generator=torch.Generator().manual_seed(tokens)).to(torch.bfloat16).cuda()
                  for inf in (768, 3072)}
            # Peak HBM footprint as the reference's stack benchmark takes it
            # (benchmarks/bench_fused_linear_stack.py:26-47): max_memory_allocated after a reset, over
            # one pass of the stack that keeps every output, each call allocating its own output and
            # scratch; latents and inputs resident.  Measured before any buffer of the timed runs
            # below exists.
            # Reported as the route's own footprint: its resident tensors (latents; x) plus what the
            # pass allocates at peak over them (outputs, scratch), so allocations elsewhere in this
            # process do not count.
            lat_mib = sum(lat.numel() * 2 for _, _, lat, _ in mats) / 2**20
            x_mib = sum(x.numel() * 2 for x in xs.values()) / 2**20
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            torch.cuda.reset_peak_memory_stats()
            before = torch.cuda.memory_allocated()
            kept = [lwl_ops.linear_forward(xs[inf], lat, outf, 3, seed, 1.0) for inf, outf, lat, seed in mats]
            torch.cuda.synchronize()
            transient = (torch.cuda.max_memory_allocated() - before) / 2**20
            row["fused_peak_MiB"] = lat_mib + x_mib + transient
            row["fused_transient_MiB"] = transient
            row["outputs_MiB"] = sum(o.numel() * 2 for o in kept) / 2**20
            del kept
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats()
            before = torch.cuda.memory_allocated()
            kept = lwl_ops.linear_forward_grouped([(xs[inf], lat, outf, 3, seed, 1.0) for inf, outf, lat, seed in mats])
            torch.cuda.synchronize()
            row["fused_grouped_peak_MiB"] = lat_mib + x_mib + (torch.cuda.max_memory_allocated() - before) / 2**20
            del kept
            # the same for the dense route: resident materialized weights, one F.linear each
            with torch.no_grad():
                ws_dense = [block_fht_slice(lat, inf * outf, 3, seed, 0, inf * outf).view(outf, inf)
                            for inf, outf, lat, seed in mats]
            torch.cuda.synchronize()
            row["dense_weights_MiB"] = sum(w.numel() * 2 for w in ws_dense) / 2**20
            torch.cuda.reset_peak_memory_stats()
            before = torch.cuda.memory_allocated()
            kept = [torch.nn.functional.linear(xs[inf], w) for (inf, _, _, _), w in zip(mats, ws_dense)]
            torch.cuda.synchronize()
            row["dense_peak_MiB"] = (x_mib + row["dense_weights_MiB"]
                                     + (torch.cuda.max_memory_allocated() - before) / 2**20)
            del kept
            outs = [torch.empty(tokens, outf, dtype=torch.bfloat16, device="cuda") for _, outf, _, _ in mats]
            wss = [abi.linear_ws(tokens, inf, outf, 32768, "cuda") for inf, outf, _, _ in mats]

            def fused_stack():
                for (inf, outf, lat, seed), o, ws in zip(mats, outs, wss):
                    abi.linear(xs[inf], lat, o, outf, 3, seed, 1.0, ws)

            def gen_stack():
                with torch.no_grad():
                    for (inf, outf, lat, seed), o in zip(mats, outs):
                        block_fht_linear_forward(xs[inf], lat, outf, 3, seed, fused=False)

            sec = time_graph(torch, gen_stack, 5, 2)
            row["generate_then_gemm_ms"] = sec * 1e3
            row["generate_then_gemm_tokens_per_s"] = tokens / sec
            if tokens == 1:
                # all 48 weights regenerated in one grouped launch (what a model-wide refresh of
                # materialized weights costs, e.g. once per optimizer step)
                specs = [(lat, inf * outf, 3, seed, 1.0, torch.bfloat16) for inf, outf, lat, seed in mats]
                wbufs = [torch.empty(inf * outf, dtype=torch.bfloat16, device="cuda") for inf, outf, _, _ in mats]
                out["grouped_regenerate_all_ms"] = time_graph(
                    torch, lambda: lwl_ops.materialize_weights(specs, wbufs), 5, 2) * 1e3
                del wbufs
            sec = time_graph(torch, fused_stack, 5, 2)
            row["fused_ms"] = sec * 1e3
            row["fused_tokens_per_s"] = tokens / sec
            # all 48 matrices in one grouped call (lwl_bfht_linear_forward_grouped): the jobs that
            # the matrix-core kernel takes below its tiled batch size share few launches; at 8192
            # tokens each job runs as its single call
            N = abi.N
            jobs = (N.LinearJob * len(mats))()
            for j, (inf, outf, lat, seed), o in zip(jobs, mats, outs):
                j.input, j.latent, j.out = xs[inf].data_ptr(), lat.data_ptr(), o.data_ptr()
                j.tokens, j.in_features, j.latent_size, j.out_features = tokens, inf, lat.numel(), outf
                j.layers, j.seed, j.weight_scale = 3, seed, 1.0
            gbytes = abi.lib.lwl_bfht_linear_forward_grouped_workspace_size(2, jobs, len(mats))
            gws = torch.empty(max(1, gbytes), dtype=torch.uint8, device="cuda")
            row["fused_grouped_workspace_MiB"] = gbytes / 2**20

            def grouped_stack():
                N.check(abi.lib.lwl_bfht_linear_forward_grouped(2, jobs, len(mats), gws.data_ptr(), gbytes,
                                                                abi.stream()))

            sec = time_graph(torch, grouped_stack, 5, 2)
            row["fused_grouped_ms"] = sec * 1e3
            row["fused_grouped_tokens_per_s"] = tokens / sec

            def dense_stack():
                for (inf, outf, _, _), o, w in zip(mats, outs, ws_dense):
                    torch.matmul(xs[inf], w.t(), out=o)

            sec = time_graph(torch, dense_stack, 5, 2)
            row["dense_ms"] = sec * 1e3
            row["dense_tokens_per_s"] = tokens / sec
            row["fused_over_dense"] = row["fused_ms"] / row["dense_ms"]
            row["fused_grouped_over_dense"] = row["fused_grouped_ms"] / row["dense_ms"]
            del ws_dense, xs, outs, wss, gws
            torch.cuda.empty_cache()
        except Exception as exc:  # noqa: BLE001
            row["error"] = f"{type(exc).__name__}: {exc}"
        out[f"tokens_{tokens}"] = row
    return out


def epilogue_bench(torch):
    from latent_weight_lab_amd import ops

    out = {}
    for tokens in (64, 4096):
        for inf, outf in ((768, 3072), (3072, 768)):
            g = torch.Generator().manual_seed(5)
            lat = torch.randn(32768, generator=g).to(torch.bfloat16).cuda()
            x = torch.randn(tokens, inf, generator=g).to(torch.bfloat16).cuda()
            bias = torch.randn(outf, generator=g).to(torch.bfloat16).cuda()
            base = torch.randn(tokens, outf, generator=g).to(torch.bfloat16).cuda()
            mod = torch.tensor([1e-3], dtype=torch.bfloat16).cuda()
            rbs = 0.5

            def fused():
                ops.linear_forward(x, lat, outf, 3, 3, rbs, bias=bias, base=base, row_sum_coef=mod,
                                   row_sum_scale=rbs)

            def sequence():
                y = ops.linear_forward(x, lat, outf, 3, 3, 1.0)
                y = y + mod * x.sum(dim=-1, keepdim=True)
                y = base + rbs * y
                y + bias

            def plain():
                ops.linear_forward(x, lat, outf, 3, 3, 1.0)

            f = time_graph(torch, fused, 20, 3)
            q = time_graph(torch, sequence, 20, 3)
            p = time_graph(torch, plain, 20, 3)
            out[f"{inf}x{outf}_tokens_{tokens}"] = {
                "fused_epilogue_ms": round(f * 1e3, 4), "sequence_ms": round(q * 1e3, 4),
                "plain_ms": round(p * 1e3, 4), "sequence_over_fused": q / f}
    return out


def mix_bench(torch):
    from latent_weight_lab_amd import ops

    def torch_mix(x, signs):  # the reference's FixedFHTMix.forward, op for op
        features = x.shape[-1]
        padded = signs.numel()
        if padded != features:
            x = torch.nn.functional.pad(x, (0, padded - features))
        out = x * signs.to(dtype=x.dtype)
        step = 1
        while step < padded:
            shape = out.shape
            out = out.reshape(*shape[:-1], -1, 2, step)
            first = out[..., 0, :].clone()
            second = out[..., 1, :].clone()
            out[..., 0, :] = first + second
            out[..., 1, :] = first - second
            out = out.reshape(shape)
            step *= 2
        out = out / math.sqrt(padded)
        return (out * signs.to(dtype=x.dtype))[..., :features]

    res = {}
    for features in (768, 3072):
        padded = 1 << (features - 1).bit_length()
        signs = (torch.randint(0, 2, (padded,), generator=torch.Generator().manual_seed(1),
                               dtype=torch.float32) * 2.0 - 1.0).cuda()
        x = torch.randn(8192, features, device="cuda").to(torch.bfloat16)
        out = torch.empty_like(x)
        nbytes = 2 * x.numel() * 2
        k = time_graph(torch, lambda: ops.fht_mix(x, signs, out=out), 50, 5)
        t = time_graph(torch, lambda: torch_mix(x, signs), 10, 2)
        res[f"8192x{features}"] = {"kernel_ms": round(k * 1e3, 5), "kernel_algo_GBs": nbytes / k / 1e9,
                                   "kernel_hbm_frac": nbytes / k / 1e9 / HBM_PEAK_GBS,
                                   "torch_reference_ms": round(t * 1e3, 4), "speedup": t / k}
    return res


def heads_bench(torch):
    from latent_weight_lab_amd import BlockFHTLinear, block_fht_grouped_input_linear, block_fht_headwise_linear

    out = {}
    cases = {
        # attention k projection per head (attn.c_attn.k_headwise): 12 x (768 -> 64), latent 492, block 2^9
        "headwise_12x768x64": (block_fht_headwise_linear, 12, 768, 64, 768),
        # MLP c_proj in 4 input groups (mlp.c_proj grouped): 4 x (768 -> 768), latent 5898, block 2^13
        "grouped_input_4x768x768": (block_fht_grouped_input_linear, 4, 768, 768, 4 * 768),
    }
    for name, (fn, nh, inf, outf, xin) in cases.items():
        torch.manual_seed(0)
        heads = [BlockFHTLinear(inf, outf, latent_ratio=0.01, layers=2, seed=1000 + i).cuda() for i in range(nh)]
        x = torch.randn(8 * 1024, xin, device="cuda").to(torch.bfloat16).requires_grad_(True)

        def per_head():
            if fn is block_fht_headwise_linear:
                y = torch.cat([h(x) for h in heads], dim=-1)
            else:
                pieces = x.split(inf, dim=-1)
                y = heads[0](pieces[0])
                for p, h in zip(pieces[1:], heads[1:]):
                    y = y + h(p)
            y.float().sum().backward()

        def batched():
            fn(x, heads).float().sum().backward()

        row = {"tokens": 8 * 1024, "heads": nh, "latent": heads[0].generator.latent.numel()}
        for tag, f in (("batched", batched), ("per_head", per_head)):
            row[tag + "_ms"] = round(time_eager(torch, f, 20, 3) * 1e3, 4)
        row["speedup"] = row["per_head_ms"] / row["batched_ms"]
        out[name] = row
        del heads, x
    return out


def cache_bench(abi, torch):
    N = abi.N
    lib = abi.lib
    mats = []
    for layer in range(12):
        for j, (inf, outf) in enumerate(GPT2_SHAPES):
            size = inf * outf
            n = max(1, round(size * 0.01))
            torch.manual_seed(1000 + 4 * layer + j)
            lat = (torch.randn(n) * 0.02).cuda()
            mats.append({"lat": lat, "size": size, "seed": 1000 + 4 * layer + j, "n": n,
                         "w32": torch.empty(size, device="cuda"),
                         "wbf": torch.empty(size, dtype=torch.bfloat16, device="cuda"),
                         "wbf2": torch.empty(size, dtype=torch.bfloat16, device="cuda"),
                         "gw": (torch.randn(size, generator=torch.Generator().manual_seed(j)) * 1e-3).to(
                             torch.bfloat16).cuda(),
                         "gl": torch.zeros(n, device="cuda"), "gl2": torch.zeros(n, device="cuda"),
                         "tmp": torch.empty(n, device="cuda")})
    for m in mats:
        m["bws"] = abi.bwd_ws(m["n"], m["size"], 0, m["size"], "cuda")
        m["g32"] = torch.empty(m["size"], device="cuda")

    def jobs(fwd):
        arr = (N.WeightJob * len(mats))()
        for j, m in zip(arr, mats):
            j.latent = m["lat"].data_ptr()
            j.weight = m["wbf"].data_ptr()
            j.grad_weight = m["gw"].data_ptr()
            j.grad_latent = m["gl"].data_ptr()
            j.latent_size, j.size, j.layers, j.seed = m["n"], m["size"], 2, m["seed"]
            j.latent_dtype, j.weight_dtype, j.weight_scale, j.accumulate = 0, 2, 1.0, int(not fwd)
        return arr

    fj, bj = jobs(True), jobs(False)
    ws_bytes = lib.lwl_bfht_flush_weight_grads_workspace_size(bj, len(mats))
    gws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")

    def grouped_prepare():
        N.check(lib.lwl_bfht_materialize_weights(fj, len(mats), abi.stream()))

    def per_module_prepare():
        for m in mats:
            abi.forward(m["lat"], m["w32"], m["size"], 2, m["seed"], 0, m["size"])
            torch.mul(m["w32"], 1.0, out=m["w32"])
            m["wbf2"].copy_(m["w32"])

    def grouped_flush():
        N.check(lib.lwl_bfht_flush_weight_grads(bj, len(mats), gws.data_ptr(), ws_bytes, abi.stream()))

    def per_module_flush():
        for m in mats:
            m["g32"].copy_(m["gw"])
            abi.backward(m["g32"], m["tmp"], m["size"], 2, m["seed"], 0, m["size"], m["bws"])
            torch.mul(m["tmp"], 1.0, out=m["tmp"])
            m["gl2"].add_(m["tmp"])

    out = {"matrices": len(mats), "params": sum(m["size"] for m in mats),
           "latent_params": sum(m["n"] for m in mats), "flush_workspace_MiB": ws_bytes / 2**20}
    fwd_bytes = sum(m["size"] * 2 + m["n"] * 4 for m in mats)
    bwd_bytes = sum(m["size"] * 2 + m["n"] * 8 for m in mats)
    for name, fn, nbytes in (("prepare_grouped", grouped_prepare, fwd_bytes),
                             ("prepare_per_module", per_module_prepare, None),
                             ("flush_grouped", grouped_flush, bwd_bytes),
                             ("flush_per_module", per_module_flush, None)):
        sec = time_graph(torch, fn, 10, 2)
        out[name + "_ms"] = round(sec * 1e3, 4)
        if nbytes:
            out[name + "_algo_GBs"] = nbytes / sec / 1e9
    out["prepare_speedup"] = out["prepare_per_module_ms"] / out["prepare_grouped_ms"]
    out["flush_speedup"] = out["flush_per_module_ms"] / out["flush_grouped_ms"]
    # the two paths agree bit for bit (same roundings; flush accumulated the same steps)
    out["prepare_bit_identical"] = all(torch.equal(m["wbf"], m["wbf2"]) for m in mats)
    out["flush_bit_identical"] = all(torch.equal(m["gl"], m["gl2"]) for m in mats)
    return out


# ---------------------------------------------------------------- CPU baseline

def cpu_baseline(gpu_out, budget_s: float = 12.0):
    """The reference's CPU fallback (block_fht_slice_torch, latent_weight_lab/block_fht.py:84-109),
    restated op for op in oracle/oracle.py, timed on this host on config 2 bf16 forward."""
    import torch

    from oracle import oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    latent = config2_latent(torch, torch.bfloat16)
    O.torch_port_slice(latent, C2_SIZE, 3, 7, 0, 2 * C2_N)  # warm-up
    times = []
    y = None
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        y = O.torch_port_slice(latent, C2_SIZE, 3, 7, 0, C2_SIZE)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end and len(times) >= 1 and times[0] > budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    # The CPU result is also a checker of the GPU output timed above; the parity that counts
    # is against the float64 C oracle (the CPU port itself runs bf16 arithmetic, as the
    # reference's fallback does on a bf16 latent).
    err = err64 = None
    if gpu_out is not None:
        got = gpu_out.float().cpu().double().numpy()
        err = O.rel_l2(got, y.double().numpy())
        try:
            from oracle import c_oracle

            err64 = O.rel_l2(got, c_oracle.forward(latent.double().numpy(), C2_SIZE, 3, 7, 0, C2_SIZE))
        except Exception as exc:  # noqa: BLE001 - reported, not fatal
            err64 = f"unavailable: {exc}"
    return {
        "value": C2_SIZE / med,
        "unit": "coords/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config 2 bf16 forward in full (256 blocks x 32768, layers 3, seed 7), torch CPU port of "
                   f"block_fht_slice_torch, median of {len(times)} runs ({med:.3f} s each); "
                   f"host {cpu_model()}, os.cpu_count()={os.cpu_count()}"),
        "gpu_vs_cpu_rel_l2": err,
        "gpu_vs_oracle_rel_l2": err64,
    }


def _median_time(fn, budget_s: float, max_runs: int = 9):
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 1 or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_extra(budget_s: float = 4.0):
    """The reference's CPU fallback on the other configurations, each timed on a bounded sample
    (median of a few runs): config 1 in full (forward, slice, backward of sum y^2 through autograd
    of the same torch ops), one 2^20 block of config 3, and config 4's fallback (materialize W
    through block_fht_slice_torch, then fp32 F.linear) on 256 tokens."""
    import torch

    from oracle import oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    res = {}
    lat = config1_latent(torch)
    sec, n = _median_time(lambda: O.torch_port_slice(lat, C1_SIZE, 3, 123, 0, C1_SIZE), budget_s)
    res["c1_fwd_f32"] = {"coords_per_s": C1_SIZE / sec, "ms": sec * 1e3, "runs": n}
    sec, n = _median_time(lambda: O.torch_port_slice(lat, C1_SIZE, 3, 123, 1000, 2000), budget_s)
    res["c1_slice_f32"] = {"coords_per_s": 1000 / sec, "ms": sec * 1e3, "runs": n}

    def c1_bwd():
        x = lat.clone().requires_grad_(True)
        O.torch_port_slice(x, C1_SIZE, 3, 123, 0, C1_SIZE).square().sum().backward()

    sec, n = _median_time(c1_bwd, budget_s)
    res["c1_fwd_bwd_f32"] = {"coords_per_s": C1_SIZE / sec, "ms": sec * 1e3, "runs": n,
                             "note": "forward + autograd backward of sum(y^2)"}
    torch.manual_seed(2)
    lat3 = torch.randn(1 << 20, dtype=torch.float32)
    sec, n = _median_time(lambda: O.torch_port_slice(lat3, 1 << 20, 3, 99, 0, 1 << 20), budget_s, 3)
    res["c3_b2^20_fwd_one_block"] = {"coords_per_s": (1 << 20) / sec, "ms": sec * 1e3, "runs": n,
                                     "note": "1 of the 64 blocks of config 3 (2^26 coords)"}
    torch.manual_seed(3)
    lat4 = torch.randn(32768, dtype=torch.float32)
    x4 = torch.randn(256, 768, dtype=torch.float32)

    def c4():
        w = O.torch_port_slice(lat4, 768 * 3072, 3, 3, 0, 768 * 3072).view(3072, 768)
        return torch.nn.functional.linear(x4, w)

    sec, n = _median_time(c4, budget_s, 5)
    res["c4_768x3072_fallback_256tok"] = {"tokens_per_s": 256 / sec, "ms": sec * 1e3, "runs": n,
                                          "note": "materialize W (72 blocks) + fp32 F.linear, 256 tokens"}
    res["cores"] = torch.get_num_threads()
    return res


# ---------------------------------------------------------------- main

def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); BlockFHT blocks "
              "shard across GPUs without communication, but no multi-GPU run is part of this build",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 64 << 20, "calls": 20}))
        return
    abi = Abi()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    settle_info = {}
    sec, gpu_out = headline(abi, args.steps, args.warmup, args.eager, settle_info)
    wall = time.perf_counter() - t0
    coords_per_s = C2_SIZE / sec
    algo_bytes = C2_SIZE * 2 + C2_N * 2
    achieved = algo_bytes / sec / 1e9
    line = {
        "metric": "generated coords/sec & % HBM roofline @ block 32768; fused-linear tokens/sec",
        "value": coords_per_s,
        "unit": "coords/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (latent ~N(0,1), torch seed 1)",
        "config": {"workload": "config 2: BlockFHT full forward, block_size 32768, 256 blocks (8,388,608 coords), "
                               "layers 3, hash seed 7, bf16 latent and output; matrix cores: bf16 operands at "
                               "each radix-32 stage, f32 accumulation",
                   "block_size": C2_N, "blocks": C2_SIZE // C2_N, "layers": C2_LAYERS, "io_dtype": "bf16",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": profiled_traffic("bfht_mfma15_fwd_c2_bf16.md")},
        "hbm_roofline_pct": 100.0 * achieved / HBM_PEAK_GBS,
        "headline_wall_s": wall,
        # untimed: the headline's own workload run for settle_s before the W warm-up steps
        "settle": settle_info or None,
    }
    if not args.no_extra:
        only = {s for s in args.only.split(",") if s}
        line["extra"] = extra_configs(abi, args.steps, args.warmup, only)
        lin = line["extra"].get("c4_linear", {})
        tok = [v.get("fused_tokens_per_s") for v in lin.values() if isinstance(v, dict) and "fused_tokens_per_s" in v]
        if tok:
            line["fused_linear_tokens_per_s"] = {k: v.get("fused_tokens_per_s") for k, v in lin.items()}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(gpu_out)
        if not args.no_extra:
            line["cpu_extra"] = cpu_extra()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
