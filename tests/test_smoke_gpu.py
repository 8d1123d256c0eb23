"""arch_probe: the code that ran was built for this GPU (the reference's tests/test_smoke.py)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_kernel_runs_native_code_for_this_gpu() -> None:
    from sparsebench_amd import _C

    out = _C.arch_probe(1000)  # not a multiple of 256: the bounds check runs
    torch.cuda.synchronize()
    major, minor = torch.cuda.get_device_capability()
    assert out.shape == (1000,)
    assert major * 100 + minor * 10 == 950, "expected an MI355X (gfx950)"
    assert torch.all(out == 950).item()


def test_rejects_bad_size() -> None:
    from sparsebench_amd import _C

    with pytest.raises(RuntimeError, match="must be positive"):
        _C.arch_probe(0)


def test_one_hip_runtime_in_process() -> None:
    from sparsebench_amd import _C

    _C.arch_probe(1)
    maps = {ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln}
    assert len(maps) == 1, maps
    libs = {ln.split()[-1] for ln in open("/proc/self/maps") if "libsparsebench_hip" in ln}
    assert len(libs) == 1, "the gfx950 library must be the one that ran"
