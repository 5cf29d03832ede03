"""ctypes binding of the C oracle (``oracle/bfht_oracle.c``) — TEST
INFRASTRUCTURE.  Used by tests and bench's checker for float64 results at full
sizes, where the numpy oracle would be slow.  Build it with ``make -C oracle``
(``__graft_entry__.build()`` does this)."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB = None
LIB_PATH = Path(__file__).resolve().parent / "lib" / "libbfht_oracle.so"


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"C oracle not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(str(LIB_PATH))
        i64, u32p, dp = ctypes.c_int64, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_double)
        L.oracle_sign_word.restype = ctypes.c_uint32
        L.oracle_sign_word.argtypes = [i64, i64, i64, i64]
        L.oracle_sign_words.restype = None
        L.oracle_sign_words.argtypes = [i64, i64, i64, i64, i64, u32p]
        L.oracle_forward.restype = ctypes.c_int
        L.oracle_forward.argtypes = [dp, i64, i64, ctypes.c_int, i64, i64, i64, dp]
        L.oracle_backward.restype = ctypes.c_int
        L.oracle_backward.argtypes = [dp, i64, i64, ctypes.c_int, i64, i64, i64, dp]
        _LIB = L
    return _LIB


def _dptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def sign_word(seed: int, block: int, layer: int, word: int) -> int:
    return int(lib().oracle_sign_word(seed, block, layer, word))


def sign_words(seed: int, block: int, layer: int, nwords: int, first_word: int = 0) -> np.ndarray:
    out = np.empty(nwords, dtype=np.uint32)
    lib().oracle_sign_words(seed, block, layer, first_word, nwords,
                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return out


def forward(latent, size: int, layers: int, seed: int, start: int, stop: int) -> np.ndarray:
    lat = np.ascontiguousarray(np.asarray(latent, dtype=np.float64))
    out = np.empty(stop - start, dtype=np.float64)
    rc = lib().oracle_forward(_dptr(lat), lat.shape[0], size, layers, seed, start, stop, _dptr(out))
    if rc != 0:
        raise ValueError(f"oracle_forward failed ({rc}) for slice [{start}, {stop}) of size {size}")
    return out


def backward(grad_out, latent_size: int, size: int, layers: int, seed: int, start: int,
             stop: int) -> np.ndarray:
    g = np.ascontiguousarray(np.asarray(grad_out, dtype=np.float64))
    out = np.empty(latent_size, dtype=np.float64)
    rc = lib().oracle_backward(_dptr(g), latent_size, size, layers, seed, start, stop, _dptr(out))
    if rc != 0:
        raise ValueError(f"oracle_backward failed ({rc})")
    return out
