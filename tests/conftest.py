"""Shared pytest setup.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; they
are the parity tests proper and call the kernels through the C ABI. The rest
run on the CPU: the oracle against its pins and golden vectors, host logic,
and that the C-ABI library loads and exports what include/ declares.
"""

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(autouse=True)
def _skip_gpu_tests_without_gpu(request: pytest.FixtureRequest) -> None:
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("needs an MI355X GPU")
