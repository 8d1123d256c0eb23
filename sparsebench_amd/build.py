"""Builds libsparsebench_hip.so in-tree with hipcc, for gfx950 only.

    python -m sparsebench_amd.build

Each .hip source is compiled to an object (in parallel) and linked into one
shared library next to this file. The tool library libsparsebench_probe.so,
not part of the C ABI, is linked on its own: the read-bandwidth probe (a
measurement tool) and CPU shims over the kernels' tile schedules (for
tests/test_tile_schedules.py). The library links libamdhip64.so.7 by
soname; inside a Python process that has imported torch, that resolves to the
HIP runtime torch already loaded, so there is one runtime per process.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
LIB_NAME = "libsparsebench_hip.so"
PROBE_LIB_NAME = "libsparsebench_probe.so"
ARCH = "gfx950"

SOURCES = ["probe.hip", "routing.hip", "sdd.hip", "dsd.hip", "combine.hip", "assigned.hip", "router.hip", "experts.hip"]
PROBE_SOURCES = ["read_probe.hip", "schedule_shims.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # Packed fp32 arithmetic stays off in all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP extension needs ROCm's hipcc to build")
    return path


def _compile(src: pathlib.Path, obj: pathlib.Path, extra: list[str]) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in proc.stderr.splitlines() if noise not in ln and ln.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err:
        print(err, file=sys.stderr)


def _link(objs: list[pathlib.Path], out: pathlib.Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{proc.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False, extra: list[str] | None = None) -> pathlib.Path:
    """Compile every source and link the shared libraries. Returns the product library's path."""
    extra = list(extra or [])
    BUILD.mkdir(exist_ok=True)
    sources = SOURCES + PROBE_SOURCES
    objs = {s: BUILD / (s.rsplit(".", 1)[0] + ".o") for s in sources}
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_compile, CSRC / s, objs[s], extra) for s in sources]
        for f in futs:
            f.result()
    out = PKG / LIB_NAME
    _link([objs[s] for s in SOURCES], out)
    _link([objs[s] for s in PROBE_SOURCES], PKG / PROBE_LIB_NAME)
    if verbose:
        print(f"built {out} and {PKG / PROBE_LIB_NAME}")
    return out


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
