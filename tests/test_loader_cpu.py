"""Loader failure on the CPU: a missing or corrupt HIP library is recorded, every entry point
that needs it raises RuntimeError naming the cause, and BlockFHT.cuda_extension_error returns
the recorded exception (reference latent_weight_lab/block_fht.py:112-146 records the
extension's load exception and :639-641 exposes it; there the fallback is the torch CPU path,
here the package has none, so the calls raise instead).

Each case runs in a fresh interpreter (the loader caches its first outcome per process) that
never initializes the GPU."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

PROBE = r"""
import json, sys
import torch
from latent_weight_lab_amd import BlockFHT, BlockFHTLinear, _native

report = {}
m = BlockFHT(16, size=40, layers=1, seed=1)
err = m.cuda_extension_error
report["error_type"] = type(err).__name__ if err is not None else None
report["error"] = str(err)
report["same_object"] = err is BlockFHTLinear(8, 12, latent_dim=8).generator.cuda_extension_error
# every C-ABI wrapper reaches the library through _native.lib() (after its device checks)
calls = {
    "lib": lambda: _native.lib(),
    "check_forward": lambda: _native.lib().lwl_bfht_check_forward(0, 16, 40, 1, 0, 40),
    "check": lambda: _native.check(_native.LWL_ERR_INVALID),
}
report["raised"] = {}
for name, call in calls.items():
    try:
        call()
        report["raised"][name] = None
    except RuntimeError as exc:
        report["raised"][name] = str(exc)
report["gpu_initialized"] = torch.cuda.is_initialized()
print("REPORT " + json.dumps(report))
"""


def run_probe(library: Path) -> dict:
    env = dict(os.environ, LWL_BFHT_LIBRARY=str(library), PYTHONPATH=str(ROOT))
    res = subprocess.run([sys.executable, "-c", PROBE], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    line = next(ln for ln in res.stdout.splitlines() if ln.startswith("REPORT "))
    return json.loads(line[len("REPORT "):])


@pytest.mark.parametrize("kind", ["missing", "corrupt"])
def test_library_load_failure_is_recorded_and_raised(tmp_path, kind):
    library = tmp_path / "liblwl_bfht.so"
    if kind == "corrupt":
        library.write_bytes(b"\x7fELF this is not a shared object" + bytes(range(256)))
    rep = run_probe(library)
    if kind == "missing":
        assert rep["error_type"] == "FileNotFoundError"
        assert str(library) in rep["error"] and "missing" in rep["error"]
    else:
        assert rep["error_type"] == "OSError"
        assert str(library) in rep["error"]
    # one recorded exception, the same object for every module
    assert rep["same_object"] is True
    for name, msg in rep["raised"].items():
        assert msg is not None, f"{name} did not raise"
        assert "library unavailable" in msg and rep["error"] in msg, (name, msg)
    assert rep["gpu_initialized"] is False
