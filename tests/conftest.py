"""Test configuration: the ``gpu`` marker and import paths for the package and the oracle."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for path in (REPO, REPO / "plm-anon_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


GOLDEN = REPO / "tests" / "golden"


def load_golden(name: str) -> dict:
    """A fixture written by tests/golden/make_golden.py: half-precision arrays come back as bf16
    tensors (they are stored as uint16 bit patterns), everything else as numpy arrays."""
    import numpy as np
    import torch

    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        out = {k: z[k] for k in z.files}
    for k in ("x", "w"):
        out[k] = torch.from_numpy(out[k].view(np.int16).copy()).view(torch.bfloat16)
    return out


def golden_names(prefix: str) -> list[str]:
    return sorted(p.stem for p in GOLDEN.glob(f"{prefix}*.npz"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda", 0)
