"""Shared pytest setup: the ``gpu`` marker and helpers.

Tests marked ``gpu`` need an MI355X and the built ``libasrattn.so``; the rest
run on the CPU.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda", torch.cuda.current_device())


def max_rel_err(out, ref) -> float:
    """max |out - ref| / max |ref|: the error relative to the reference's
    magnitude (element-wise relative error is undefined near zero)."""
    import torch

    out = torch.as_tensor(out).double().cpu()
    ref = torch.as_tensor(ref).double().cpu()
    scale = ref.abs().max().clamp(min=1e-30)
    return float((out - ref).abs().max() / scale)
