import os
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
def force_tile():
    """Force the GEMM tile shape for the duration of a test (HXMI_GEMM_TILE)."""
    old = os.environ.get("HXMI_GEMM_TILE")

    def _set(t):
        if t is None:
            os.environ.pop("HXMI_GEMM_TILE", None)
        else:
            os.environ["HXMI_GEMM_TILE"] = str(t)

    yield _set
    if old is None:
        os.environ.pop("HXMI_GEMM_TILE", None)
    else:
        os.environ["HXMI_GEMM_TILE"] = old
