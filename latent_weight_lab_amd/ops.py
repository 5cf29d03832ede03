"""Tensor-level calls into the HIP library.

Each function validates devices/dtypes, allocates outputs and scratch through
torch's caching allocator, and launches on the current stream of the
tensors' device.  Nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as N


def _device_guard(device: torch.device):
    return torch.cuda.device(device)


def next_power_of_two(value: int) -> int:
    """Reference ``block_fht.py:12-15``."""
    if value <= 0:
        raise ValueError("value must be positive")
    return 1 << (int(value) - 1).bit_length()


def forward(latent: torch.Tensor, size: int, layers: int, seed: int, start: int, stop: int) -> torch.Tensor:
    """Generated coordinates ``[start, stop)`` (reference ext.forward,
    ``csrc/block_fht_ext_cuda.cu:516-566``)."""
    dev = N.require_cuda(latent)
    latent = latent.contiguous()
    code = N.dtype_code(latent.dtype)
    L = N.lib()
    n = latent.numel()
    N.check(L.lwl_bfht_check_forward(code, n, size, layers, start, stop))
    out = torch.empty(stop - start, dtype=latent.dtype, device=dev)
    if stop == start:
        return out
    with _device_guard(dev):
        ws_ptr, ws_size, ws = N.workspace(L.lwl_bfht_forward_workspace_size(n, size, start, stop), dev)
        N.check(L.lwl_bfht_forward(latent.data_ptr(), code, n, size, layers, seed, start, stop,
                                   out.data_ptr(), ws_ptr, ws_size, N.stream_ptr(dev)))
    del ws
    return out


def backward(grad_out: torch.Tensor, latent_size: int, latent_dtype: torch.dtype, size: int, layers: int,
             seed: int, start: int, stop: int) -> torch.Tensor:
    """Latent gradient of the slice (reference ext.backward,
    ``csrc/block_fht_ext_cuda.cu:568-622``), summed over blocks in a fixed order."""
    dev = N.require_cuda(grad_out)
    grad_out = grad_out.contiguous().to(dtype=latent_dtype)
    if grad_out.numel() != stop - start:
        raise N.BlockFHTArgumentError(
            f"grad_out has {grad_out.numel()} elements, slice [{start}, {stop}) needs {stop - start}")
    code = N.dtype_code(latent_dtype)
    L = N.lib()
    grad_latent = torch.empty(latent_size, dtype=latent_dtype, device=dev)
    with _device_guard(dev):
        ws_ptr, ws_size, ws = N.workspace(L.lwl_bfht_backward_workspace_size(latent_size, size, start, stop), dev)
        N.check(L.lwl_bfht_backward(grad_out.data_ptr() if grad_out.numel() else 0, code, latent_size, size,
                                    layers, seed, start, stop, grad_latent.data_ptr(), ws_ptr, ws_size,
                                    N.stream_ptr(dev)))
    del ws
    return grad_latent


def linear_supported(in_features: int, out_features: int, latent: torch.Tensor, x: torch.Tensor) -> bool:
    """Whether the fused kernel takes this shape (else the caller materializes)."""
    if not (x.is_cuda and latent.is_cuda and x.dtype == latent.dtype and x.dtype in N.DTYPE_CODES):
        return False
    return N.lib().lwl_bfht_check_linear_forward(N.dtype_code(x.dtype), max(1, x.numel() // max(1, in_features)),
                                                 in_features, latent.numel(), out_features, 1) == N.LWL_OK


# Batches from these sizes on run faster as W generated once plus a GEMM than through the
# fused kernels (MI355X, graph-replayed calls): the bf16 block-2^15 kernel at GPT-2 shapes
# 12.5-20.8 against 14.8-18.5 us at 128 tokens and 1.1-1.8x slower from 256; the reference
# domain (1024 -> 4096, latent 16384) 12.5-12.9 against 17.7-23.5 us at one token, about even
# at 8, slower from 32.
FUSED_MAX_TOKENS_MFMA15 = 128
FUSED_MAX_TOKENS_SMALL = 8


def linear_fused_preferred(in_features: int, out_features: int, latent: torch.Tensor, x: torch.Tensor) -> bool:
    """Whether the default route of the linear forward takes the fused kernel: it takes
    the shape and the batch is below the size from which generating W once and calling a
    GEMM is faster (the fused kernels then pay for regenerating W per token range and,
    from 256 tokens, for a re-laid-out copy of x that outweighs the transient W)."""
    if not linear_supported(in_features, out_features, latent, x):
        return False
    tokens = x.numel() // max(1, in_features)
    mfma15 = latent.dtype == torch.bfloat16 and next_power_of_two(latent.numel()) == 32768
    return tokens < (FUSED_MAX_TOKENS_MFMA15 if mfma15 else FUSED_MAX_TOKENS_SMALL)


def _epilogue(tokens: int, out_features: int, dtype: torch.dtype, dev, bias=None, base=None,
              row_sum_coef=None, row_sum_scale: float = 1.0):
    """The ``lwl_bfht_linear_epilogue`` of the given terms (None: no epilogue) and the
    tensors it points to (to keep alive until the launch is queued)."""
    if bias is None and base is None and row_sum_coef is None:
        return None, []
    ep, keep = N.LinearEpilogue(), []
    if bias is not None:
        if bias.dtype != dtype or bias.numel() != out_features or bias.device != dev:
            raise N.BlockFHTArgumentError(f"fused linear bias must be {out_features} values of {dtype} on {dev}")
        bias = bias.contiguous()
        ep.bias = bias.data_ptr()
        keep.append(bias)
    if base is not None:
        if base.dtype != dtype or tuple(base.shape) != (tokens, out_features) or base.device != dev:
            raise N.BlockFHTArgumentError(f"fused linear base must be a [{tokens}, {out_features}] {dtype} on {dev}")
        base = base.contiguous()
        ep.base = base.data_ptr()
        keep.append(base)
    if row_sum_coef is not None:
        coef = row_sum_coef.detach().reshape(1).to(device=dev, dtype=torch.float32)
        ep.row_sum_coef = coef.data_ptr()
        ep.row_sum_scale = float(row_sum_scale)
        keep.append(coef)
    return ep, keep


def linear_forward(x2d: torch.Tensor, latent: torch.Tensor, out_features: int, layers: int, seed: int,
                   weight_scale: float, bias: torch.Tensor | None = None, base: torch.Tensor | None = None,
                   row_sum_coef: torch.Tensor | None = None, row_sum_scale: float = 1.0) -> torch.Tensor:
    """Fused ``x @ (weight_scale * W)^T`` with W generated on chip (reference
    ext.linear_forward, ``csrc/block_fht_ext_cuda.cu:624-681``).  With any of ``bias``
    ``[out]``, ``base`` ``[tokens, out]`` (both of x's dtype) or ``row_sum_coef`` (a device
    scalar) the kernels' stores form ``((weight_scale * x W^T + row_sum_scale * row_sum_coef *
    x.sum(-1)) + base) + bias`` in float32, in that order, before the one rounding
    (``lwl_bfht_linear_forward_ex``; the order of the reference ``forward_fused``'s tail,
    ``block_fht.py:493-500``)."""
    dev = N.require_cuda(x2d, latent)
    x2d = x2d.contiguous()
    latent = latent.contiguous()
    code = N.dtype_code(x2d.dtype)
    if latent.dtype != x2d.dtype:
        raise RuntimeError("block_fht_linear_forward: input and latent dtype must match")
    tokens, in_features = x2d.shape
    L = N.lib()
    N.check(L.lwl_bfht_check_linear_forward(code, tokens, in_features, latent.numel(), out_features, layers))
    out = torch.empty(tokens, out_features, dtype=x2d.dtype, device=dev)
    if tokens == 0:
        return out
    ep, keep = _epilogue(tokens, out_features, x2d.dtype, dev, bias, base, row_sum_coef, row_sum_scale)
    epp = ctypes.byref(ep) if ep is not None else None
    with _device_guard(dev):
        need = L.lwl_bfht_linear_forward_ex_workspace_size(code, tokens, in_features, out_features, latent.numel(), epp)
        ws_ptr, ws_size, ws = N.workspace(need, dev)
        N.check(L.lwl_bfht_linear_forward_ex(x2d.data_ptr(), latent.data_ptr(), code, tokens, in_features,
                                             latent.numel(), out_features, layers, seed, float(weight_scale), epp,
                                             out.data_ptr(), ws_ptr, ws_size, N.stream_ptr(dev)))
    del ws, keep
    return out


def linear_forward_grouped(specs: list[tuple], outs: list[torch.Tensor] | None = None) -> list[torch.Tensor]:
    """Many fused linears ``x @ (weight_scale * W)^T`` in few launches
    (``lwl_bfht_linear_forward_grouped``); each result equals its own ``linear_forward`` call
    bit for bit.  ``specs``: ``(x2d, latent, out_features, layers, seed, weight_scale)`` per
    matrix, all of one dtype, optionally followed by a dict of ``linear_forward``'s epilogue
    arguments (``bias``, ``base``, ``row_sum_coef``, ``row_sum_scale``); ``outs``: optional
    preallocated ``[tokens, out_features]`` outputs."""
    if not specs:
        return []
    dev = N.require_cuda(*[t for sp in specs for t in sp[:2]])
    dtype = specs[0][0].dtype
    code = N.dtype_code(dtype)
    jobs, result, keep, epis = [], [], [], []
    for i, spec in enumerate(specs):
        x2d, latent, out_features, layers, seed, scale = spec[:6]
        extra = spec[6] if len(spec) > 6 and spec[6] else {}
        x2d = x2d.contiguous()
        latent = latent.contiguous()
        if x2d.dtype != dtype or latent.dtype != dtype:
            raise RuntimeError("grouped fused linear: every input and latent must have the same dtype")
        tokens, in_features = x2d.shape
        if outs is None:
            out = torch.empty(tokens, int(out_features), dtype=dtype, device=dev)
        else:
            out = outs[i]
            if out.shape != (tokens, int(out_features)) or out.dtype != dtype or not out.is_contiguous():
                raise N.BlockFHTArgumentError(f"output {i} must be a contiguous [{tokens}, {out_features}] {dtype}")
        j = N.LinearJob()
        j.input, j.latent, j.out = x2d.data_ptr(), latent.data_ptr(), out.data_ptr()
        j.tokens, j.in_features, j.latent_size = tokens, in_features, latent.numel()
        j.out_features, j.layers, j.seed, j.weight_scale = int(out_features), int(layers), int(seed), float(scale)
        ep, ep_keep = _epilogue(tokens, int(out_features), dtype, dev, **extra)
        if ep is not None:
            j.epilogue = ctypes.pointer(ep)
            epis.append(ep)
            keep += ep_keep
        jobs.append(j)
        result.append(out)
        keep += [x2d, latent]
    arr = (N.LinearJob * len(jobs))(*jobs)
    L = N.lib()
    N.check(L.lwl_bfht_check_linear_jobs(code, arr, len(jobs)))
    with _device_guard(dev):
        ws_ptr, ws_size, ws = N.workspace(L.lwl_bfht_linear_forward_grouped_workspace_size(code, arr, len(jobs)), dev)
        N.check(L.lwl_bfht_linear_forward_grouped(code, arr, len(jobs), ws_ptr, ws_size, N.stream_ptr(dev)))
    del ws, keep, epis
    return result


def linear_backward_latent_supported(in_features: int, out_features: int, latent: torch.Tensor,
                                     x: torch.Tensor, grad: torch.Tensor) -> bool:
    """Whether the fused latent gradient takes this shape (else grad_weight is formed in HBM)."""
    if not (x.is_cuda and latent.is_cuda and grad.is_cuda and x.dtype == latent.dtype == grad.dtype
            and x.dtype in N.DTYPE_CODES):
        return False
    tokens = max(1, x.numel() // max(1, in_features))
    return N.lib().lwl_bfht_check_linear_backward_latent(N.dtype_code(x.dtype), tokens, in_features,
                                                         latent.numel(), out_features, 1) == N.LWL_OK


def linear_backward_latent(grad2d: torch.Tensor, x2d: torch.Tensor, latent: torch.Tensor, out_features: int,
                           layers: int, seed: int, weight_scale: float) -> torch.Tensor:
    """``weight_scale * block_fht_grad_latent(latent, (grad2d^T x2d).flatten(), ...)`` in one library
    call: the weight gradient on the library's split-K matrix-core GEMM (float32 partials in the
    workspace), then the generator's backward (the grad_latent branch of the reference's
    ``_BlockFHTLinearFn.backward``, ``block_fht.py:339-350``; the modulation term is the caller's)."""
    dev = N.require_cuda(grad2d, x2d, latent)
    grad2d = grad2d.contiguous()
    x2d = x2d.contiguous()
    code = N.dtype_code(latent.dtype)
    if not (grad2d.dtype == x2d.dtype == latent.dtype):
        raise RuntimeError("linear latent gradient: grad, input and latent dtype must match")
    tokens, in_features = x2d.shape
    if grad2d.shape != (tokens, out_features):
        raise ValueError(f"grad shape {tuple(grad2d.shape)} does not match ({tokens}, {out_features})")
    L = N.lib()
    N.check(L.lwl_bfht_check_linear_backward_latent(code, tokens, in_features, latent.numel(), out_features,
                                                    layers))
    grad_latent = torch.empty(latent.numel(), dtype=latent.dtype, device=dev)
    with _device_guard(dev):
        need = L.lwl_bfht_linear_backward_latent_workspace_size(tokens, in_features, out_features, latent.numel())
        ws_ptr, ws_size, ws = N.workspace(need, dev)
        N.check(L.lwl_bfht_linear_backward_latent(grad2d.data_ptr() if tokens else 0, x2d.data_ptr() if tokens else 0,
                                                  code, tokens, in_features, latent.numel(), out_features, layers,
                                                  seed, float(weight_scale), grad_latent.data_ptr(), ws_ptr,
                                                  ws_size, N.stream_ptr(dev)))
    del ws
    return grad_latent


def _weight_job(latent: torch.Tensor, size: int, layers: int, seed: int, weight_scale: float,
                weight_dtype: torch.dtype) -> N.WeightJob:
    j = N.WeightJob()
    j.latent = latent.data_ptr()
    j.latent_size = latent.numel()
    j.size = int(size)
    j.layers = int(layers)
    j.seed = int(seed)
    j.latent_dtype = N.dtype_code(latent.dtype)
    j.weight_dtype = N.dtype_code(weight_dtype)
    j.weight_scale = float(weight_scale)
    return j


def _job_array(jobs: list) -> ctypes.Array:
    return (N.WeightJob * max(1, len(jobs)))(*jobs)


def weight_job_supported(latent: torch.Tensor, size: int, layers: int, weight_dtype: torch.dtype,
                         grad_weight: torch.Tensor | None = None) -> bool:
    """Whether the grouped weight-cache kernels take this generator (host-only check;
    the pointers are not dereferenced).  Without ``grad_weight`` the materialize
    side is checked, with it the flush side."""
    if not latent.is_cuda or latent.dtype not in N.DTYPE_CODES or weight_dtype not in N.DTYPE_CODES:
        return False
    if not latent.is_contiguous():
        return False
    j = _weight_job(latent, size, layers, 0, 1.0, weight_dtype)
    if grad_weight is None:
        j.weight = j.latent
        forward = 1
    else:
        if not grad_weight.is_cuda or not grad_weight.is_contiguous() or grad_weight.dtype != weight_dtype:
            return False
        j.grad_weight = grad_weight.data_ptr()
        j.grad_latent = j.latent
        forward = 0
    return N.lib().lwl_bfht_check_weight_jobs(_job_array([j]), 1, forward) == N.LWL_OK


def materialize_weights(specs: list[tuple], outs: list[torch.Tensor] | None = None) -> list[torch.Tensor]:
    """Generate whole weights of many generators in a few launches (the per-module
    ``materialize_weight_cache`` calls of the reference's ``prepare_block_fht_weight_cache``,
    ``block_fht.py:503-563``).

    ``specs``: ``(latent, size, layers, seed, weight_scale, weight_dtype)`` per generator.
    Returns flat weights equal to ``(generate(latent) * weight_scale).to(weight_dtype)``,
    written into ``outs`` (contiguous, ``size`` elements of ``weight_dtype`` each) when given.
    """
    if not specs:
        return []
    dev = N.require_cuda(*[s[0] for s in specs])
    if outs is not None and len(outs) != len(specs):
        raise N.BlockFHTArgumentError("outs must match specs")
    jobs, result, keep = [], [], []
    for i, (latent, size, layers, seed, weight_scale, weight_dtype) in enumerate(specs):
        latent = latent.detach().contiguous()
        if outs is None:
            out = torch.empty(int(size), dtype=weight_dtype, device=dev)
        else:
            out = outs[i]
            if (out.dtype != weight_dtype or out.numel() != int(size) or not out.is_contiguous()
                    or out.device != dev):
                raise N.BlockFHTArgumentError(f"output {i} must be a contiguous {weight_dtype} tensor of {size}")
        j = _weight_job(latent, size, layers, seed, weight_scale, weight_dtype)
        j.weight = out.data_ptr()
        jobs.append(j)
        result.append(out)
        keep.append(latent)
    L = N.lib()
    arr = _job_array(jobs)
    with _device_guard(dev):
        N.check(L.lwl_bfht_materialize_weights(arr, len(jobs), N.stream_ptr(dev)))
    return result


def flush_weight_grads(specs: list[tuple]) -> list[torch.Tensor]:
    """Project many weight gradients back onto their latents in a few launches (the
    per-module ``flush_weight_cache_to_latent_grad`` calls of the reference's
    ``flush_block_fht_weight_cache``, ``block_fht.py:514-569``).

    ``specs``: ``(latent, grad_weight, size, layers, seed, weight_scale, into)`` per
    generator; ``into`` is None or a contiguous tensor of the latent's shape and dtype
    that the result is added to in place (``latent.grad.add_``).  Returns, per spec,
    ``into`` or a new tensor holding ``weight_scale * block_fht_grad_latent(latent,
    grad_weight.to(latent.dtype), ...)``.
    """
    if not specs:
        return []
    dev = N.require_cuda(*[s[1] for s in specs])
    jobs, outs, keep = [], [], []
    for latent, grad_weight, size, layers, seed, weight_scale, into in specs:
        grad_weight = grad_weight.detach().contiguous()
        if grad_weight.numel() != size:
            raise N.BlockFHTArgumentError(f"grad_weight has {grad_weight.numel()} elements, size is {size}")
        if into is None:
            out = torch.empty(latent.numel(), dtype=latent.dtype, device=dev)
        else:
            if into.dtype != latent.dtype or into.numel() != latent.numel() or not into.is_contiguous():
                raise N.BlockFHTArgumentError("accumulation target must be a contiguous tensor like the latent")
            out = into
        j = _weight_job(latent, size, layers, seed, weight_scale, grad_weight.dtype)
        j.grad_weight = grad_weight.data_ptr()
        j.grad_latent = out.data_ptr()
        j.accumulate = int(into is not None)
        jobs.append(j)
        outs.append(out)
        keep.append(grad_weight)
    L = N.lib()
    arr = _job_array(jobs)
    with _device_guard(dev):
        ws_ptr, ws_size, ws = N.workspace(L.lwl_bfht_flush_weight_grads_workspace_size(arr, len(jobs)), dev)
        N.check(L.lwl_bfht_flush_weight_grads(arr, len(jobs), ws_ptr, ws_size, N.stream_ptr(dev)))
    del ws, keep
    return outs


def sign_words(seed: int, block: int, layer: int, nwords: int, first_word: int = 0,
               device: torch.device | str = "cuda") -> torch.Tensor:
    """Sign words computed by the device hash (int32 tensor holding the uint32 bits)."""
    device = torch.device(device)
    out = torch.empty(nwords, dtype=torch.int32, device=device)
    with _device_guard(device):
        N.check(N.lib().lwl_bfht_sign_words(seed, block, layer, first_word, nwords,
                                            ctypes.cast(out.data_ptr(), ctypes.POINTER(ctypes.c_uint32)),
                                            N.stream_ptr(device)))
    return out


def fht_mix(x: torch.Tensor, signs: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``(S H S pad(x))[..., :features]`` over the last dimension (``FixedFHTMix.forward``,
    reference ``examples/nanogpt/model.py:200-218``); ``signs`` holds ±1 for the padded
    length.  ``out`` may be ``x`` (in place)."""
    dev = N.require_cuda(x, signs)
    features = int(x.shape[-1])
    padded = next_power_of_two(features)
    if signs.numel() != padded:
        raise N.BlockFHTArgumentError(f"signs must hold {padded} values for {features} features")
    signs = signs.detach().to(dtype=torch.float32).contiguous()
    x = x.contiguous()
    rows = x.numel() // features if features else 0
    code = N.dtype_code(x.dtype)
    L = N.lib()
    N.check(L.lwl_fht_check_mix(code, rows, features))
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise N.BlockFHTArgumentError("out must be a contiguous tensor like x")
    with _device_guard(dev):
        N.check(L.lwl_fht_mix(x.data_ptr(), code, rows, features, signs.data_ptr(), out.data_ptr(),
                              N.stream_ptr(dev)))
    return out
