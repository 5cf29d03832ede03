"""ctypes binding of ``liblwl_bfht.so`` (C ABI in ``include/lwl_bfht.h``).

PyTorch supplies device memory and the current HIP stream; every computation
runs in the HIP library.  There is no CPU fallback: if the library cannot be
loaded, every entry point raises with the loader's error.

The library must share torch's HIP runtime (torch ships its own
``libamdhip64.so``), so torch is imported before the library is opened; the
library's ``libamdhip64.so.7`` dependency then resolves to the copy torch
already mapped (same SONAME), and streams and device pointers interoperate.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_NAME = "liblwl_bfht.so"

# status codes (include/lwl_bfht.h)
LWL_OK = 0
LWL_ERR_INVALID = -1
LWL_ERR_UNSUPPORTED = -2
LWL_ERR_WORKSPACE = -3
LWL_ERR_HIP = -4

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


class WeightJob(ctypes.Structure):
    """``lwl_bfht_weight_job``: one module's whole weight in a grouped
    materialize / flush call."""
    _fields_ = [
        ("latent", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("grad_weight", ctypes.c_void_p),
        ("grad_latent", ctypes.c_void_p),
        ("latent_size", ctypes.c_int64),
        ("size", ctypes.c_int64),
        ("layers", ctypes.c_int64),
        ("seed", ctypes.c_int64),
        ("latent_dtype", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("weight_scale", ctypes.c_double),
        ("accumulate", ctypes.c_int32),
    ]


class LinearEpilogue(ctypes.Structure):
    """``lwl_bfht_linear_epilogue``: out = ((weight_scale * x @ W^T + row_sum_scale *
    (*row_sum_coef) * x.sum(-1)) + base) + bias in float32 in that order, one rounding."""
    _fields_ = [
        ("bias", ctypes.c_void_p),
        ("base", ctypes.c_void_p),
        ("row_sum_coef", ctypes.c_void_p),
        ("row_sum_scale", ctypes.c_double),
    ]


class LinearJob(ctypes.Structure):
    """``lwl_bfht_linear_job``: one matrix of a grouped fused-linear call."""
    _fields_ = [
        ("input", ctypes.c_void_p),
        ("latent", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("tokens", ctypes.c_int64),
        ("in_features", ctypes.c_int64),
        ("latent_size", ctypes.c_int64),
        ("out_features", ctypes.c_int64),
        ("layers", ctypes.c_int64),
        ("seed", ctypes.c_int64),
        ("weight_scale", ctypes.c_double),
        ("epilogue", ctypes.POINTER(LinearEpilogue)),
    ]


class BlockFHTArgumentError(ValueError, RuntimeError):
    """Invalid argument.  The reference raises ValueError from its Python
    checks and RuntimeError from its extension's TORCH_CHECKs; this is both."""


_lock = threading.Lock()
_lib = None
_error: Exception | None = None


def library_path() -> Path:
    override = os.environ.get("LWL_BFHT_LIBRARY")
    return Path(override) if override else LIB_DIR / LIB_NAME


def _bind(lib) -> None:
    i64, i32, sz, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
    dbl, u32p = ctypes.c_double, ctypes.POINTER(ctypes.c_uint32)
    jobp = ctypes.POINTER(WeightJob)
    ljobp = ctypes.POINTER(LinearJob)
    epip = ctypes.POINTER(LinearEpilogue)
    sigs = {
        "lwl_last_error": (ctypes.c_char_p, []),
        "lwl_abi_version": (i32, []),
        "lwl_bfht_forward_workspace_size": (sz, [i64, i64, i64, i64]),
        "lwl_bfht_forward": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, vp, vp, sz, vp]),
        "lwl_bfht_check_forward": (i32, [i32, i64, i64, i64, i64, i64]),
        "lwl_bfht_backward_workspace_size": (sz, [i64, i64, i64, i64]),
        "lwl_bfht_backward": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, vp, vp, sz, vp]),
        "lwl_bfht_backward_noalloc": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, vp, vp]),
        "lwl_bfht_linear_forward_workspace_size": (sz, [i64, i64, i64, i64]),
        "lwl_bfht_linear_forward": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, dbl, vp, vp, sz, vp]),
        "lwl_bfht_check_linear_forward": (i32, [i32, i64, i64, i64, i64, i64]),
        "lwl_bfht_linear_forward_ex_workspace_size": (sz, [i32, i64, i64, i64, i64, epip]),
        "lwl_bfht_linear_forward_ex": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, dbl, epip, vp, vp, sz, vp]),
        "lwl_bfht_check_linear_jobs": (i32, [i32, ljobp, i64]),
        "lwl_bfht_linear_forward_grouped_workspace_size": (sz, [i32, ljobp, i64]),
        "lwl_bfht_linear_forward_grouped": (i32, [i32, ljobp, i64, vp, sz, vp]),
        "lwl_bfht_linear_backward_latent_workspace_size": (sz, [i64, i64, i64, i64]),
        "lwl_bfht_linear_backward_latent": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, dbl, vp, vp, sz, vp]),
        "lwl_bfht_check_linear_backward_latent": (i32, [i32, i64, i64, i64, i64, i64]),
        "lwl_bfht_sign_words": (i32, [i64, i64, i64, i64, i64, u32p, vp]),
        "lwl_bfht_check_weight_jobs": (i32, [jobp, i64, i32]),
        "lwl_bfht_materialize_weights": (i32, [jobp, i64, vp]),
        "lwl_bfht_flush_weight_grads_workspace_size": (sz, [jobp, i64]),
        "lwl_bfht_flush_weight_grads": (i32, [jobp, i64, vp, sz, vp]),
        "lwl_fht_mix": (i32, [vp, i32, i64, i64, vp, vp, vp]),
        "lwl_fht_check_mix": (i32, [i32, i64, i64]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """The loaded library; raises RuntimeError (with the cause) if it cannot load."""
    global _lib, _error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None and _error is None:
            try:
                path = library_path()
                if not path.exists():
                    raise FileNotFoundError(
                        f"{path} is missing; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                        " or `python -m latent_weight_lab_amd.build`")
                handle = ctypes.CDLL(str(path))
                _bind(handle)
                _lib = handle
            except Exception as exc:  # noqa: BLE001 - recorded and re-raised below
                _error = exc
    if _lib is None:
        raise RuntimeError(f"latent_weight_lab_amd: HIP BlockFHT library unavailable: {_error}") from _error
    return _lib


def load_error() -> Exception | None:
    """The exception that prevented loading, if any (reference API:
    ``BlockFHT.cuda_extension_error``, block_fht.py:639-641)."""
    try:
        lib()
    except RuntimeError:
        pass
    return _error


def check(rc: int) -> None:
    if rc == LWL_OK:
        return
    msg = lib().lwl_last_error().decode("utf-8", "replace")
    if rc == LWL_ERR_INVALID:
        raise BlockFHTArgumentError(msg)
    raise RuntimeError(f"latent_weight_lab_amd: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(
            f"latent_weight_lab_amd: BlockFHT supports float32, float16 and bfloat16, got {dtype}") from None


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> tuple[int, int, torch.Tensor | None]:
    """(pointer, size, owner) of a scratch buffer from torch's caching allocator."""
    if nbytes == 0:
        return 0, 0, None
    buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return buf.data_ptr(), nbytes, buf


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "latent_weight_lab_amd runs BlockFHT on the GPU only; move the latent and inputs "
                "to a cuda device (this package has no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"latent_weight_lab_amd: tensors on different devices ({dev}, {t.device})")
    return dev
