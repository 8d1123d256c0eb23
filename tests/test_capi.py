"""The C-ABI library without a GPU: it loads (with torch's HIP runtime), exports
every entry point include/sparsebench_hip.h declares, and its host-side
argument checks and size arithmetic agree with the oracle. No kernel runs.
"""

import ctypes
import pathlib
import re

import pytest

from oracle.topology_ref import worst_case_sizes
from sparsebench_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from sparsebench_amd.build import build

        build()
    return _lib.lib()


def declared_functions() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(sb_\w+)\s*\(", text))
    return names


def test_header_declares_the_path() -> None:
    assert {"sb_routing", "sb_sdd", "sb_dsd", "sb_combine", "sb_arch_probe"} <= declared_functions()


def test_library_exports_every_declared_symbol(lib) -> None:
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_one_hip_runtime_in_process(lib) -> None:
    maps = {ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln}
    assert len(maps) == 1, maps


def test_version(lib) -> None:
    assert lib.sb_version() == 1


def _err(lib) -> str:
    return lib.sb_last_error().decode()


def test_arch_probe_rejects_non_positive(lib) -> None:
    assert lib.sb_arch_probe(None, 0, None) == 1
    assert "must be positive" in _err(lib)


@pytest.mark.parametrize("num_copies", [1, 26, 2000, 8192, 200_000])
@pytest.mark.parametrize("num_experts", [1, 8, 64, 1024])
@pytest.mark.parametrize("block_size", [4, 128])
def test_routing_sizes_match_oracle(lib, num_copies: int, num_experts: int, block_size: int) -> None:
    rb, rows, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    rc = lib.sb_routing_sizes(num_copies, num_experts, 2 * block_size, block_size,
                              ctypes.byref(rb), ctypes.byref(rows), ctypes.byref(ws))
    assert rc == 0, _err(lib)
    assert (rb.value, rows.value) == worst_case_sizes(num_copies, num_experts, 2 * block_size, block_size)
    # The host wrapper sizes the workspace itself: it must agree with the library.
    assert ws.value == (num_copies + 1023) // 1024 * (num_experts + 1)


@pytest.mark.parametrize(
    ("args", "match"),
    [
        ((10, 0, 32, 16), "num_experts"),
        ((10, 2000, 32, 16), "num_experts"),
        ((10, 8, 30, 16), "multiple"),
        ((10, 8, 32, 0), "block_size"),
        ((2**30, 1024, 2**20, 128), "too large"),
    ],
)
def test_routing_sizes_reject(lib, args, match: str) -> None:
    assert lib.sb_routing_sizes(*args, None, None, None) == 1
    assert match in _err(lib)


def test_dsd_rejects_block_size(lib) -> None:
    assert lib.sb_dsd(None, None, None, None, None, 1, 128, 1, 32, 256, 0, None) == 1
    assert "64 or 128" in _err(lib)


def test_dsd_rejects_d(lib) -> None:
    assert lib.sb_dsd(None, None, None, None, None, 1, 128, 1, 64, 100, 0, None) == 1
    assert "multiple of 128" in _err(lib)


def test_sdd_rejects_shapes(lib) -> None:
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    assert lib.sb_sdd(p, p, p, p, p, p, 4, 96, 256, 2, 1, 1, None) == 1
    assert "multiple of 64" in _err(lib)
    assert lib.sb_sdd(p, p, p, p, p, p, 4, 128, 128, 2, 1, 1, None) == 1
    assert "multiple of 256" in _err(lib)


def test_combine_rejects_gate_dtype(lib) -> None:
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    assert lib.sb_combine(p, p, p, 7, p, 1, 2, 8, 4, None, None) == 1
    assert "gate dtype" in _err(lib)


def test_combines_reject_more_than_2_31_workgroups(lib) -> None:
    # One lane per 16 bytes of output, 256 lanes per workgroup: the grid of
    # ceil(T * D / 8 / 256) workgroups must stay below 2^31.
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    assert lib.sb_combine(p, p, p, 0, p, 1 << 36, 2, 64, 4, None, None) == 1
    assert "too many tokens" in _err(lib)
    assert lib.sb_combine_assigned(p, p, p, 0, p, None, p, 1 << 36, 64, 4, None, None) == 1
    assert "too many tokens" in _err(lib)


@pytest.mark.parametrize(("num_tokens", "num_experts", "k", "tile"),
                         [(4096, 64, 2, 128), (50, 3, 1, 4), (16384, 128, 2, 128), (1000, 65, 3, 16)])
def test_router_sizes(lib, num_tokens: int, num_experts: int, k: int, tile: int) -> None:
    cap, rb, rows, ws = (ctypes.c_int64() for _ in range(4))
    rc = lib.sb_router_sizes(num_tokens, num_experts, k, tile, 128, 512, ctypes.byref(cap), ctypes.byref(rb),
                             ctypes.byref(rows), ctypes.byref(ws))
    assert rc == 0, _err(lib)
    # An expert rounds up by less than half a tile; never more than T*E assignments.
    assert cap.value == min(num_tokens * num_experts, num_tokens * k + num_experts * (tile // 2))
    assert (rb.value, rows.value) == worst_case_sizes(cap.value, num_experts, 512, 128)
    words, chunks = (num_tokens + 31) // 32, (num_tokens + 63) // 64
    assert ws.value == chunks * num_experts + num_experts + num_tokens * num_experts + 2 * words * num_experts \
        + 2 * num_tokens


@pytest.mark.parametrize(("args", "match"), [
    ((0, 8, 2, 128), "T > 0"), ((10, 0, 2, 128), "num_experts"), ((10, 2000, 2, 128), "num_experts"),
    ((10, 8, 0, 128), "k must be"), ((10, 8, 9, 128), "k must be"), ((100, 64, 17, 128), "k must be"),
    ((10, 8, 2, 0), "tile"),
])
def test_router_sizes_reject(lib, args, match: str) -> None:
    assert lib.sb_router_sizes(*args, 128, 256, None, None, None, None) == 1
    assert match in _err(lib)


def test_router_entry_points_reject_null_buffers(lib) -> None:
    assert lib.sb_router_topk(None, 10, 8, 2, None, None, None) == 1
    assert "null buffer" in _err(lib)
    assert lib.sb_token_rounding(None, 10, 8, 2, 128, 128, 256, *([None] * 15)) == 1
    assert "null buffer" in _err(lib)


def test_assigned_entry_points_reject(lib) -> None:
    assert lib.sb_routing_assigned(None, 0, None, 0, 0, 10, 8, 256, 128, None, *([None] * 10)) == 1
    assert "must not be empty" in _err(lib)
    assert lib.sb_routing_assigned(None, 0, None, 0, 5, 10, 8, 256, 128, None, *([None] * 10)) == 1
    assert "null buffer" in _err(lib)
    assert lib.sb_token_csr(None, 0, None, 5, 0, None, None, None) == 1
    assert "token count" in _err(lib)
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    assert lib.sb_combine_assigned(p, p, p, 9, p, None, p, 1, 8, 4, None, None) == 1
    assert "weight dtype" in _err(lib)
    assert lib.sb_combine_assigned(p, p, p, 2, p, None, p, 1, 12, 4, None, None) == 1
    assert "multiple of 8" in _err(lib)


def test_test_hooks_set_and_reject(lib) -> None:
    assert lib.sb_set_test_hook(0, 1) == 0
    assert lib.sb_set_test_hook(0, 0) == 0
    assert lib.sb_set_test_hook(1, 0) == 0
    assert lib.sb_set_test_hook(2, 1) == 1
    assert "unknown test hook" in _err(lib)
    assert lib.sb_set_test_hook(-1, 1) == 1

