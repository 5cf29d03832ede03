"""The ctypes shim that INTEGRATION.md (Option B) gives a maintainer of the reference to put in
place of ``_load_block_fht_ext`` (reference latent_weight_lab/block_fht.py:116-146): the three
methods of the reference extension (``csrc/block_fht_ext.cpp:69-73``) over this build's C ABI.
Kept here verbatim so that the tests exercise exactly the binding the document shows."""
from __future__ import annotations

import ctypes

import torch


class _LwlExt:
    _DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

    def __init__(self, path):
        L = ctypes.CDLL(path)
        i64, i32, sz, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
        L.lwl_last_error.restype = ctypes.c_char_p
        L.lwl_bfht_forward_workspace_size.restype = sz
        L.lwl_bfht_forward_workspace_size.argtypes = [i64, i64, i64, i64]
        L.lwl_bfht_forward.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, vp, vp, sz, vp]
        L.lwl_bfht_backward_workspace_size.restype = sz
        L.lwl_bfht_backward_workspace_size.argtypes = [i64, i64, i64, i64]
        L.lwl_bfht_backward.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, vp, vp, sz, vp]
        L.lwl_bfht_linear_forward_workspace_size.restype = sz
        L.lwl_bfht_linear_forward_workspace_size.argtypes = [i64, i64, i64, i64]
        L.lwl_bfht_linear_forward.argtypes = [vp, vp, i32, i64, i64, i64, i64, i64, i64, ctypes.c_double,
                                              vp, vp, sz, vp]
        self.L = L

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.L.lwl_last_error().decode())

    def _ws(self, nbytes, dev):
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
        return (buf.data_ptr() if buf is not None else 0), nbytes, buf

    def forward(self, latent, size, layers, seed, start, stop):
        out = torch.empty(stop - start, dtype=latent.dtype, device=latent.device)
        p, n, keep = self._ws(self.L.lwl_bfht_forward_workspace_size(latent.numel(), size, start, stop),
                              latent.device)
        self._check(self.L.lwl_bfht_forward(latent.data_ptr(), self._DT[latent.dtype], latent.numel(), size,
                                            layers, seed, start, stop, out.data_ptr(), p, n,
                                            torch.cuda.current_stream().cuda_stream))
        return [out]

    def backward(self, grad_out, latent_size, size, layers, seed, start, stop):
        g = torch.empty(latent_size, dtype=grad_out.dtype, device=grad_out.device)
        p, n, keep = self._ws(self.L.lwl_bfht_backward_workspace_size(latent_size, size, start, stop),
                              grad_out.device)
        self._check(self.L.lwl_bfht_backward(grad_out.data_ptr(), self._DT[grad_out.dtype], latent_size, size,
                                             layers, seed, start, stop, g.data_ptr(), p, n,
                                             torch.cuda.current_stream().cuda_stream))
        return g

    def linear_forward(self, input, latent, out_features, layers, seed, weight_scale):
        tokens, in_features = input.shape
        out = torch.empty(tokens, out_features, dtype=input.dtype, device=input.device)
        p, n, keep = self._ws(self.L.lwl_bfht_linear_forward_workspace_size(tokens, in_features, out_features,
                                                                           latent.numel()), input.device)
        self._check(self.L.lwl_bfht_linear_forward(input.data_ptr(), latent.data_ptr(), self._DT[input.dtype],
                                                   tokens, in_features, latent.numel(), out_features, layers,
                                                   seed, weight_scale, out.data_ptr(), p, n,
                                                   torch.cuda.current_stream().cuda_stream))
        return out
