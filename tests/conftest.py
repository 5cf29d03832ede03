from __future__ import annotations

import base64
import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN_PATH = ROOT / "tests" / "golden" / "bfht_golden.json"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


def decode_array(value):
    """Fixture arrays are ``"f8:<base64>"`` / ``"f4:<base64>"`` little-endian."""
    if isinstance(value, str) and value[:3] in ("f8:", "f4:"):
        dtype = "<" + value[:2]
        return np.frombuffer(base64.b64decode(value[3:]), dtype=dtype).astype(np.float64)
    return np.asarray(value, dtype=np.float64)


@pytest.fixture(scope="session")
def golden():
    return json.loads(GOLDEN_PATH.read_text())


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False
