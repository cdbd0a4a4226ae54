"""Test configuration: the ``gpu`` marker and import paths.

``sigmod-kvscope_amd/`` is put on ``sys.path`` so the drop-in modules import under the
reference's names (``runtime.audit_kernel``, ``observe.tile_shares``, ``runtime.block_view``),
and the repository root so ``oracle`` imports.
"""

import json
import math
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sigmod-kvscope_amd")
for path in (PKG, ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def _decode(value):
    if isinstance(value, str) and value in ("nan", "inf", "-inf"):
        return float(value)
    if isinstance(value, list):
        return [_decode(v) for v in value]
    if isinstance(value, dict):
        return {k: _decode(v) for k, v in value.items()}
    return value


def load_golden(name: str) -> dict:
    """A fixture from tests/golden, with "nan" / "inf" / "-inf" strings turned into floats."""
    with open(os.path.join(GOLDEN, name)) as f:
        return _decode(json.load(f))


def as_array(value, dtype=np.float64) -> np.ndarray:
    return np.array(value, dtype=dtype)


@pytest.fixture(scope="session")
def known_answers() -> dict:
    return load_golden("known_answers.json")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip():
    """The loaded HIP library; GPU tests fail (not skip) when it is missing."""
    import ekv_hip

    return ekv_hip.load()


def close(a, b, tol) -> bool:
    return math.isclose(a, b, abs_tol=tol)
