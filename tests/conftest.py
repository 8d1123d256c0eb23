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


class LayerHooks:
    """The library's test hooks and moe_forward's stage choices for one test
    (restored when it ends): each forces a code path whose output must not
    differ from the built-in choice's."""

    def __init__(self) -> None:
        self._stage: dict[str, bool] | None = None

    def expert_gate(self, value) -> None:
        """1: the layer kernels' expert tiles, 2: their row blocks, 0: the device's choice."""
        from sparsebench_amd import _C

        _C.set_test_hook("expert_gate", int(value))

    def topk_kernel(self, value) -> None:
        """1: the top-k router's wave form, 2: its lane form, 0: the built-in choice."""
        from sparsebench_amd import _C

        _C.set_test_hook("topk_kernel", int(value))

    def stage(self, **options: bool) -> None:
        """moe.set_stage_options(expert_tiles=...)."""
        from sparsebench_amd import moe

        previous = moe.set_stage_options(**options)
        if self._stage is None:
            self._stage = previous

    def restore(self) -> None:
        from sparsebench_amd import _C, moe

        for name in ("expert_gate", "topk_kernel"):
            _C.set_test_hook(name, 0)
        if self._stage is not None:
            moe.set_stage_options(**self._stage)


@pytest.fixture
def hooks():
    h = LayerHooks()
    yield h
    h.restore()
