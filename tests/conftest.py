import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "miraclereasoning-cpu_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

GOLDEN = Path(__file__).resolve().parent / "golden"

# One-line results of parity tests that the pass/fail status does not show
# (near-ties adopted in discrete choices), printed in the session's summary.
_NOTES = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture(scope="session")
def backend():
    """One HIPBackend for the whole GPU session (the reference's tests share one
    OpenCL backend the same way, tests/conftest.py:8-17)."""
    from miracle_hip import HIPBackend
    return HIPBackend()


@pytest.fixture
def parity_note():
    return _NOTES.append


def pytest_terminal_summary(terminalreporter):
    if _NOTES:
        terminalreporter.write_sep("-", "parity notes")
        for line in _NOTES:
            terminalreporter.write_line(line)
