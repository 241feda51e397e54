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



# Element-wise parity, beside the normwise bound max|out - ref| / max|ref|
# <= rtol: every element must satisfy
#     |out - ref| <= rtol * (|ref| + atol),   atol = ATOL_FRACTION * rms(ref).
# The floor atol keeps near-zero reference elements (where a relative error
# has no meaning) from deciding the result; per tolerance class it is a
# stated multiple of the reference's root-mean-square value.  For elements
# smaller than the typical one this bound is stricter than the normwise
# one (whose absolute allowance is rtol * max|ref|, about 4 rms).  Measured
# on the full GPU suite, the worst element reaches 0.61 (f32), 0.76 (bf16)
# and 0.40 (module) of its bound.
ATOL_FRACTION = {"f32": 2.0, "bf16": 1.0, "module": 0.25}
RTOL = {"f32": 1e-5, "bf16": 2e-2}
_RECORDS = []


def elementwise_err(out, ref, atol_fraction: float) -> float:
    """max |out - ref| / (|ref| + atol) with atol = atol_fraction * rms(ref)."""
    import torch

    out = torch.as_tensor(out).double().cpu()
    ref = torch.as_tensor(ref).double().cpu()
    atol = atol_fraction * float(ref.pow(2).mean().sqrt().clamp(min=1e-30))
    return float(((out - ref).abs() / (ref.abs() + atol)).max())


def assert_close(out, ref, kind: str, rtol: float | None = None, label: str = "") -> None:
    """Both parity bounds, normwise (max_rel_err) and element-wise
    (elementwise_err with the class's atol), each at most rtol (default
    RTOL[kind]; the "module" class, outputs that include GEMMs, takes rtol
    explicitly)."""
    rtol = RTOL[kind] if rtol is None else rtol
    norm = max_rel_err(out, ref)
    elem = elementwise_err(out, ref, ATOL_FRACTION[kind])
    _RECORDS.append((kind, norm / rtol, elem / rtol))
    assert norm <= rtol, f"{label} normwise error {norm:.3g} > {rtol:g}"
    assert elem <= rtol, f"{label} element-wise error {elem:.3g} > {rtol:g} (atol {ATOL_FRACTION[kind]} rms)"


def pytest_terminal_summary(terminalreporter, exitstatus, config) -> None:
    """The worst parity figures of the run, per tolerance class."""
    if not _RECORDS:
        return
    worst = {}
    for kind, norm, elem in _RECORDS:
        w = worst.setdefault(kind, [0.0, 0.0, 0])
        w[0], w[1], w[2] = max(w[0], norm), max(w[1], elem), w[2] + 1
    terminalreporter.write_line("parity (worst error / bound, per tolerance class):")
    for kind, (norm, elem, count) in sorted(worst.items()):
        terminalreporter.write_line(
            f"  {kind}: {count} checks, normwise {norm:.3f}, element-wise {elem:.3f} (atol {ATOL_FRACTION[kind]} rms)"
        )
