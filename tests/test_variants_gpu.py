"""Every SDD / DSD tile variant compiled into the library against the oracle.

The library picks one variant per shape; SPARSEBENCH_SDD_VARIANT /
SPARSEBENCH_DSD_VARIANT select any other (for tuning). All must give the
oracle's results to the same bf16 tolerance as the defaults (1.6e-2).
"""

import math

import pytest
import torch

from oracle.moe_ref import dsd_rows, sdd_blocks
from oracle.topology_ref import build_layout
from sparsebench_amd.workloads import routing_case

pytestmark = pytest.mark.gpu

TOL = {"rtol": 1.6e-2, "atol": 1.6e-2}
COMMON = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 21, 22, 23, 24, 25, 26, 27, 31, 32, 33, 34,
          35, 36, 37, 38, 39, 51, 52, 53, 54, 55, 56, 57, 58, 59, 61, 62, 63, 64, 65]
SDD_PERSISTENT = [41, 43, 44]
DSD_PERSISTENT = [41, 42, 43, 44, 45]
SDD_VARIANTS = COMMON + SDD_PERSISTENT
DSD_VARIANTS = COMMON + DSD_PERSISTENT


@pytest.mark.parametrize("variant", SDD_VARIANTS)
@pytest.mark.parametrize("case", ["zipf", "empty_middle"])
def test_sdd_variant(monkeypatch, variant: int, case: str) -> None:
    from sparsebench_amd.routing import route_device
    from sparsebench_amd.spmm import sdd

    monkeypatch.setenv("SPARSEBENCH_SDD_VARIANT", str(variant))
    g = torch.Generator().manual_seed(variant)
    e, d, f, t = 8, 256, 512, 600
    idx = routing_case(case, t, e, seed=variant)
    x = torch.randn(t, d, generator=g).bfloat16()
    w1 = (torch.randn(e, d, f, generator=g) / d**0.5).bfloat16()
    dev = route_device(idx.cuda(), e, f, 128)
    out = sdd(x.cuda(), w1.cuda(), dev)
    lay = build_layout(idx.numpy(), e, f, 128)
    torch.testing.assert_close(out[: lay.col_indices.size].float().cpu(), sdd_blocks(x.float(), w1.float(), lay),
                               **TOL)


@pytest.mark.parametrize("variant", DSD_VARIANTS)
@pytest.mark.parametrize("bs", [64, 128])
def test_dsd_variant(monkeypatch, variant: int, bs: int) -> None:
    from sparsebench_amd import _C

    monkeypatch.setenv("SPARSEBENCH_DSD_VARIANT", str(variant))
    g = torch.Generator().manual_seed(100 + variant)
    e, f, d = 8, 2 * bs, 512
    lay = build_layout(routing_case("zipf", 500, e, seed=variant).numpy(), e, f, bs)
    blocks = (torch.randn(lay.col_indices.size, bs, bs, generator=g) / math.sqrt(f)).bfloat16()
    w = torch.randn(e * f, d, generator=g).bfloat16()
    out = _C.dsd_cuda(blocks.cuda(), w.cuda(), torch.as_tensor(lay.row_offsets).cuda(),
                      torch.as_tensor(lay.col_indices).cuda(), 4)
    torch.testing.assert_close(out.float().cpu(), dsd_rows(blocks.float(), w.float(), lay), **TOL)


# The persistent forms run about one workgroup per CU slot (256 on MI355X),
# each walking several tiles with the DMA ring crossing tile boundaries.
# These shapes give 2-6 tiles per workgroup, tiles of different experts in a
# row, and dead row blocks after the live ones (worst-case buffers).


@pytest.mark.parametrize("variant", SDD_PERSISTENT)
@pytest.mark.parametrize("case", ["random", "zipf_perm"])
def test_sdd_persistent_many_tiles(monkeypatch, variant: int, case: str) -> None:
    from sparsebench_amd.routing import route_device
    from sparsebench_amd.spmm import sdd

    monkeypatch.setenv("SPARSEBENCH_SDD_VARIANT", str(variant))
    g = torch.Generator().manual_seed(variant)
    e, d, f, t = 64, 256, 1536, 4096
    idx = routing_case(case, t, e, seed=variant)
    x = torch.randn(t, d, generator=g).bfloat16()
    w1 = (torch.randn(e, d, f, generator=g) / d**0.5).bfloat16()
    dev = route_device(idx.cuda(), e, f, 128)
    out = sdd(x.cuda(), w1.cuda(), dev)
    lay = build_layout(idx.numpy(), e, f, 128)
    torch.testing.assert_close(out[: lay.col_indices.size].float().cpu(), sdd_blocks(x.float(), w1.float(), lay),
                               **TOL)


@pytest.mark.parametrize("variant", DSD_PERSISTENT)
@pytest.mark.parametrize("version", [1, 4])
def test_dsd_persistent_many_tiles(monkeypatch, variant: int, version: int) -> None:
    from sparsebench_amd.routing import route_device
    from sparsebench_amd.spmm import dsd

    monkeypatch.setenv("SPARSEBENCH_DSD_VARIANT", str(variant))
    g = torch.Generator().manual_seed(200 + variant)
    e, f, d, bs, t = 64, 256, 2048, 128, 4096
    idx = routing_case("zipf_perm", t, e, seed=variant)
    dev = route_device(idx.cuda(), e, f, bs)
    blocks = (torch.randn(dev.col_indices.numel(), bs, bs, generator=g) / math.sqrt(f)).bfloat16()
    w = torch.randn(e * f, d, generator=g).bfloat16()
    out = dsd(blocks.cuda(), w.cuda(), dev, version=version)
    lay = build_layout(idx.numpy(), e, f, bs)
    torch.testing.assert_close(out[: lay.num_rows].float().cpu(), dsd_rows(blocks.float(), w.float(), lay), **TOL)
    if version == 1:  # zeroes dead row blocks
        assert torch.all(out[lay.num_rows:] == 0)


@pytest.mark.parametrize("group", ["1", "3", "8", "64"])
def test_tile_group_orders_agree(monkeypatch, group: str) -> None:
    # The tile order changes which workgroup computes which tile, not the math:
    # results are bit-identical for every group size.
    from sparsebench_amd.moe import moe_forward

    g = torch.Generator().manual_seed(7)
    t, e, d, f = 700, 16, 256, 512
    x = torch.randn(t, d, generator=g).bfloat16().cuda()
    w1 = (torch.randn(e, d, f, generator=g) / d**0.5).bfloat16().cuda()
    w2 = (torch.randn(e, f, d, generator=g) / f**0.5).bfloat16().cuda()
    idx = routing_case("zipf", t, e).cuda()
    gates = torch.rand(t, 2, generator=g).cuda()
    monkeypatch.delenv("SPARSEBENCH_TILE_GROUP", raising=False)
    ref = moe_forward(x, idx, gates, w1, w2)
    monkeypatch.setenv("SPARSEBENCH_TILE_GROUP", group)
    assert torch.equal(moe_forward(x, idx, gates, w1, w2), ref)
