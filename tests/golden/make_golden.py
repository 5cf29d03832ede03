"""Write the golden input/output vectors for the BlockFHT path.

This script runs ONLY in the build container, where the reference checkout is
mounted at ``/root/reference``.  It imports the reference's pure-PyTorch CPU
path (``latent_weight_lab/block_fht.py``; nothing from it is compiled or run on
a GPU) and records, in float64, what that code returns for small seeded inputs:

* ``sign_word_for`` (``block_fht.py:46-52``): the only part of the path whose
  constants and mixing order no mathematical identity pins;
* ``signs_for`` (``block_fht.py:55-81``): the word/bit layout of the signs;
* ``block_fht_slice_torch`` (``block_fht.py:84-109``): the composition order of
  signs and normalized FHTs, slicing across blocks, zero padding;
* the autograd backward of that function (``block_fht.py:180-196``);
* ``block_fht_linear_forward`` fallback (``block_fht.py:251-288``): the
  ``W[o, i] = flat[o * in + i]`` view and the ``weight_scale`` placement.

The vectors go to ``bfht_golden.json`` beside this file.  Tests read only that
JSON file; they never import the reference.
"""
from __future__ import annotations

import base64
import json
import sys
from pathlib import Path

import torch

REFERENCE = Path("/root/reference")


def _load_reference():
    sys.path.insert(0, str(REFERENCE))
    from latent_weight_lab import block_fht as ref  # noqa: E402

    return ref


def _f64_list(t: torch.Tensor) -> str:
    """Little-endian bytes, base64: exact and compact.  float32 tensors stay f4."""
    code = "f4" if t.dtype == torch.float32 else "f8"
    arr = t.detach().to(torch.float32 if code == "f4" else torch.float64).reshape(-1).numpy()
    return code + ":" + base64.b64encode(arr.astype("<" + code).tobytes()).decode("ascii")


def main() -> None:
    ref = _load_reference()
    torch.set_num_threads(1)
    out: dict = {"source": "latent_weight_lab/block_fht.py (reference CPU path, float64)"}

    # --- sign words -------------------------------------------------------
    seeds = [0, 1, 7, 99, 123, 999, -1, -2, -123456789, 2**32 + 5, 2**40 + 3,
             -(2**33) - 7, 2**63 - 1, -(2**63)]
    blocks = [0, 1, 2, 255, 1000, 2**31 + 3, 2**32 - 1]
    layers = [0, 1, 2, 3]
    words = [0, 1, 31, 1023, 262143]
    sw = []
    for s in seeds:
        for b in blocks:
            for l in layers:
                for w in words:
                    sw.append([s, b, l, w, ref.sign_word_for(s, b, l, w)])
    out["sign_words"] = sw

    # --- sign vectors -----------------------------------------------------
    sv = []
    for (seed, block, layer, bs) in [(999, 3, 2, 65), (123, 0, 0, 8), (7, 5, 1, 32),
                                     (-5, 17, 3, 100), (2**35 + 9, 2, 2, 64), (0, 0, 0, 1)]:
        sig = ref.signs_for(torch.empty(1, dtype=torch.float64), block, layer, seed, bs)
        sv.append({"seed": seed, "block": block, "layer": layer, "block_size": bs,
                   "signs": [int(v) for v in sig.tolist()]})
    out["signs"] = sv

    # --- forward / backward slices ---------------------------------------
    cases = []

    def add_case(name, latent, size, L, seed, start, stop, full_samples=None, grad_stride=1):
        lat = latent.to(torch.float64).clone().requires_grad_(True)
        y = ref.block_fht_slice_torch(lat, size, L, seed, start, stop)
        y.square().sum().backward()
        case = {
            "name": name, "latent": _f64_list(latent), "size": size,
            "layers": L, "seed": seed, "start": start, "stop": stop,
            "out": _f64_list(y),
        }
        if grad_stride == 1:
            case["grad_sumsq"] = _f64_list(lat.grad)
        else:
            case["grad_sumsq_stride"] = grad_stride
            case["grad_sumsq_sampled"] = _f64_list(lat.grad[::grad_stride])
            case["grad_sumsq_sum"] = float(lat.grad.sum())
            case["grad_sumsq_sumsq"] = float(lat.grad.square().sum())
        if full_samples is not None:
            with torch.no_grad():
                full = ref.block_fht_slice_torch(latent.to(torch.float64), size, L, seed, 0, size)
            idx = list(range(0, size, full_samples)) + [size - 1]
            case["full_sum"] = float(full.sum())
            case["full_sumsq"] = float(full.square().sum())
            case["full_sample_index"] = idx
            case["full_sample_value"] = [float(full[i]) for i in idx]
        cases.append(case)

    g = torch.Generator().manual_seed(42)
    # reference tests: tests/test_block_fht.py:34-46, 62-67
    add_case("ref_test_slice_n7", torch.randn(7, generator=g, dtype=torch.float64), 31, 2, 123, 3, 17)
    add_case("ref_test_full_n7", torch.randn(7, generator=g, dtype=torch.float64), 31, 2, 123, 0, 31)
    add_case("ref_test_function_n8", torch.randn(8, generator=g, dtype=torch.float64), 40, 2, 7, 5, 23)
    add_case("b64_negative_seed", torch.randn(40, generator=g, dtype=torch.float64), 1000, 1, -5, 50, 333)
    add_case("b32_exact_l3", torch.randn(32, generator=g, dtype=torch.float64), 96, 3, 2**33 + 1, 0, 96)
    add_case("b1_tiny", torch.randn(1, generator=g, dtype=torch.float64), 5, 3, 11, 0, 5)
    add_case("b256_l3_ragged", torch.randn(200, generator=g, dtype=torch.float64), 1500, 3, 77, 255, 1290)
    add_case("empty_slice", torch.randn(16, generator=g, dtype=torch.float64), 64, 2, 3, 20, 20)
    # torch.manual_seed(0) randn(1024) fp32, size 108618, layers 3, seed 123
    torch.manual_seed(0)
    c1 = torch.randn(1024, dtype=torch.float32)
    add_case("config1_slice_1000_2000", c1, 108_618, 3, 123, 1000, 2000, full_samples=997)
    # tests/test_block_fht_cuda.py:30-31 shape (global-memory backend in the reference)
    torch.manual_seed(0)
    big = torch.randn(20000, dtype=torch.float32)
    add_case("ref_cuda_global_n20000", big, 65536, 1, 123, 111, 4096, grad_stride=13)
    out["slices"] = cases

    # --- linear -----------------------------------------------------------
    lin = []
    g = torch.Generator().manual_seed(7)
    for (inf, outf, n, L, seed, scale, tokens) in [(5, 3, 8, 2, 11, 1.0, 4), (7, 5, 32, 2, 99, 1.0, 11),
                                                   (12, 10, 50, 3, 5, 0.125, 6), (8, 6, 32, 1, 7, 0.5, 5),
                                                   (40, 3, 16, 2, -3, 2.0, 3)]:
        latent = torch.randn(n, generator=g, dtype=torch.float64)
        x = torch.randn(tokens, inf, generator=g, dtype=torch.float64)
        y = ref.block_fht_linear_forward(x, latent, outf, L, seed, weight_scale=scale)
        lin.append({"in_features": inf, "out_features": outf, "latent": _f64_list(latent),
                    "layers": L, "seed": seed, "weight_scale": scale, "x": _f64_list(x),
                    "tokens": tokens, "out": _f64_list(y)})
    out["linear"] = lin

    path = Path(__file__).with_name("bfht_golden.json")
    path.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
