import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no GPU is visible")
    return torch.device("cuda:0")


@pytest.fixture
def knobs(pkg):
    """Launch-shape overrides (hxmi_set_tuning) for the duration of a test:
    knobs(gemm_tile=3, splitk=4, ...); None clears one."""
    saved = {}

    def _set(**kw):
        for name, value in kw.items():
            prev = pkg.set_tuning(name, value)
            saved.setdefault(name, prev)

    yield _set
    for name, prev in saved.items():
        pkg.set_tuning(name, prev)


@pytest.fixture
def force_tile(knobs):
    """Force the GEMM tile shape (TileId) for the duration of a test."""
    return lambda t: knobs(gemm_tile=t)
