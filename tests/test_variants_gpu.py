"""Every tile form the SDD / DSD drop-ins pick, against the oracle.

sb_sdd / sb_dsd pick one tile form per shape (sdd_tile_for in sdd_tile.hpp,
dispatch_dsd in dsd.hip). These tests reach each of them through the shape
that selects it, for both block sizes of the DSD, and hold it to the bf16
tolerance of the defaults (1.6e-2):

  SDD  128 x 512, 3 stages (D < 4096, F % 512 == 0)   D 256, F 512
       128 x 512, 4 stages (D >= 4096)                 D 4096, F 512
       128 x 256 (F % 512 != 0)                        D 256, F 768
  DSD  512 wide, 4 waves (D % 512 == 0, K < 8192)      D 512, K 256
       512 wide, 8 waves (K = F per expert >= 8192)    D 512, K 8192
       256 wide (D % 512 != 0, D % 256 == 0)           D 768
       128 wide (D % 256 != 0)                         D 384
"""

import math

import pytest
import torch

from oracle.moe_ref import dsd_rows, sdd_blocks
from oracle.topology_ref import build_layout
from sparsebench_amd.workloads import routing_case

pytestmark = pytest.mark.gpu

TOL = {"rtol": 1.6e-2, "atol": 1.6e-2}


@pytest.mark.parametrize(("d_model", "ffn_dim"), [(256, 512), (4096, 512), (256, 768)], ids=["wide", "deep", "narrow"])
@pytest.mark.parametrize("case", ["zipf", "empty_middle"])
def test_sdd_tile_forms(d_model: int, ffn_dim: int, case: str) -> None:
    from sparsebench_amd.routing import route_device
    from sparsebench_amd.spmm import sdd

    g = torch.Generator().manual_seed(d_model + ffn_dim)
    e, t = 8, 600
    idx = routing_case(case, t, e, seed=3)
    x = torch.randn(t, d_model, generator=g).bfloat16()
    w1 = (torch.randn(e, d_model, ffn_dim, generator=g) / d_model**0.5).bfloat16()
    dev = route_device(idx.cuda(), e, ffn_dim, 128)
    out = sdd(x.cuda(), w1.cuda(), dev)
    lay = build_layout(idx.numpy(), e, ffn_dim, 128)
    torch.testing.assert_close(out[: lay.col_indices.size].float().cpu(), sdd_blocks(x.float(), w1.float(), lay),
                               **TOL)


@pytest.mark.parametrize(("d_model", "ffn_dim"), [(512, 256), (512, 8192), (768, 256), (384, 256)],
                         ids=["wide", "deep_k", "mid", "narrow"])
@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("version", [1, 4])
def test_dsd_tile_forms(d_model: int, ffn_dim: int, bs: int, version: int) -> None:
    from sparsebench_amd import _C

    g = torch.Generator().manual_seed(100 + d_model + bs)
    e = 8
    t = 300 if ffn_dim > 1024 else 500
    lay = build_layout(routing_case("zipf", t, e, seed=5).numpy(), e, ffn_dim, bs)
    blocks = (torch.randn(lay.col_indices.size, bs, bs, generator=g) / math.sqrt(ffn_dim)).bfloat16()
    w = torch.randn(e * ffn_dim, d_model, generator=g).bfloat16()
    # Worst-case buffers: two dead row blocks after the live ones.
    row_offsets = torch.cat([torch.as_tensor(lay.row_offsets), torch.full((2,), int(lay.row_offsets[-1]))]).int()
    out = _C.dsd_cuda(blocks.cuda(), w.cuda(), row_offsets.cuda(), torch.as_tensor(lay.col_indices).cuda(), version)
    torch.testing.assert_close(out[: lay.num_rows].float().cpu(), dsd_rows(blocks.float(), w.float(), lay), **TOL)
    if version == 1:  # versions 1-3 write dead row blocks as zeros
        assert torch.all(out[lay.num_rows:] == 0)
