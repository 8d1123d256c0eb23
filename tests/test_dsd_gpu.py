"""DSD (BSR @ dense) against the fp32 block-wise oracle, for every version code
of the reference (tests/test_dsd.py there). One gfx950 kernel serves all the
codes; they differ only in whether dead row blocks are zeroed and in v5's
shape limits, so the full case grid runs for one code of each behaviour and
a smaller grid for the rest.

Tolerance: rtol = atol = 1.6e-2 (bf16 output rounding), as in the reference.
"""

import math

import pytest
import torch

from oracle.moe_ref import bsr_to_dense, dsd_rows
from oracle.topology_ref import build_layout
from sparsebench_amd.workloads import CASE_NAMES, routing_case

pytestmark = pytest.mark.gpu

ALL_VERSIONS = (1, 2, 21, 3, 31, 4, 41, 5)
ZEROS_DEAD_ROWS = {1, 2, 21, 3, 31}
TOL = {"rtol": 1.6e-2, "atol": 1.6e-2}


def supports(version: int, bs: int, d_model: int) -> bool:
    return version != 5 or (bs == 128 and d_model % 256 == 0)


def make_inputs(case, num_tokens, num_experts, ffn_dim, d_model, bs, seed=0):
    g = torch.Generator().manual_seed(seed)
    lay = build_layout(routing_case(case, num_tokens, num_experts, seed).numpy(), num_experts, ffn_dim, bs)
    blocks = (torch.randn(lay.col_indices.size, bs, bs, generator=g) / math.sqrt(ffn_dim)).bfloat16()
    w = torch.randn(num_experts * ffn_dim, d_model, generator=g).bfloat16()
    return lay, blocks, w


def run(blocks, w, lay, version):
    from sparsebench_amd import _C

    ro = torch.as_tensor(lay.row_offsets).cuda()
    ci = torch.as_tensor(lay.col_indices).cuda()
    return _C.dsd_cuda(blocks.cuda(), w.cuda(), ro, ci, version)


def oracle(blocks, w, lay):
    return dsd_rows(blocks.float(), w.float(), lay)


def test_oracle_matches_dense_reference() -> None:
    lay, blocks, w = make_inputs("zipf", 50, 4, 128, 128, 64)
    torch.testing.assert_close(oracle(blocks, w, lay), bsr_to_dense(blocks.float(), lay) @ w.float(),
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("version", [1, 4, 5])
@pytest.mark.parametrize("case", CASE_NAMES)
@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize(("num_experts", "f_blocks"), [(8, 1), (8, 4), (64, 1), (64, 2), (8, 3)],
                         ids=["E8F1", "E8F4", "E64F1", "E64F2", "E8F3"])
@pytest.mark.parametrize("d_model", [128, 256, 512], ids=["D128", "D256", "D512"])
def test_matches_oracle(version, case, bs, num_experts, f_blocks, d_model) -> None:
    if not supports(version, bs, d_model):
        pytest.skip(f"v{version} does not take bs={bs}, D={d_model}")
    lay, blocks, w = make_inputs(case, 300, num_experts, f_blocks * bs, d_model, bs)
    torch.testing.assert_close(run(blocks, w, lay, version).float().cpu(), oracle(blocks, w, lay), **TOL)


@pytest.mark.parametrize("version", [2, 21, 3, 31, 41])
@pytest.mark.parametrize("case", ["random", "zipf"])
@pytest.mark.parametrize("bs", [64, 128])
def test_other_version_codes(version, case, bs) -> None:
    lay, blocks, w = make_inputs(case, 300, 8, 2 * bs, 256, bs)
    torch.testing.assert_close(run(blocks, w, lay, version).float().cpu(), oracle(blocks, w, lay), **TOL)


@pytest.mark.parametrize("version", ALL_VERSIONS)
@pytest.mark.parametrize("bs", [64, 128])
def test_single_token(version, bs) -> None:
    if not supports(version, bs, 256):
        pytest.skip(f"v{version} does not take bs={bs}")
    lay, blocks, w = make_inputs("random", 1, 8, 2 * bs, 256, bs)
    torch.testing.assert_close(run(blocks, w, lay, version).float().cpu(), oracle(blocks, w, lay), **TOL)


@pytest.mark.parametrize("version", ALL_VERSIONS)
@pytest.mark.parametrize("bs", [64, 128])
def test_asymmetric_inputs(version, bs) -> None:
    if not supports(version, bs, 256):
        pytest.skip(f"v{version} does not take bs={bs}")
    lay, _, _ = make_inputs("random", 200, 8, 2 * bs, 256, bs)
    k_total, d_model = 8 * 2 * bs, 256
    i = torch.arange(k_total, dtype=torch.float32)[:, None]
    j = torch.arange(d_model, dtype=torch.float32)[None, :]
    w = torch.sin(0.37 * i + 1.31 * j + 0.05 * i * j / d_model).bfloat16()
    p = torch.arange(lay.col_indices.size, dtype=torch.float32)[:, None, None]
    r = torch.arange(bs, dtype=torch.float32)[None, :, None]
    c = torch.arange(bs, dtype=torch.float32)[None, None, :]
    blocks = (torch.cos(0.7 * r - 0.23 * c + 0.11 * p + 0.01 * r * c) / math.sqrt(2 * bs)).bfloat16()
    torch.testing.assert_close(run(blocks, w, lay, version).float().cpu(), oracle(blocks, w, lay), **TOL)


@pytest.mark.parametrize("version", ALL_VERSIONS)
def test_worst_case_device_topology(version) -> None:
    from sparsebench_amd.routing import route_device
    from sparsebench_amd.spmm import dsd

    bs, num_experts, ffn_dim, d_model = 128, 64, 256, 256
    idx = routing_case("zipf", 400, num_experts)
    dev = route_device(idx.cuda(), num_experts, ffn_dim, bs)
    g = torch.Generator().manual_seed(3)
    blocks = (torch.randn(dev.col_indices.numel(), bs, bs, generator=g) / 16).bfloat16()
    w = torch.randn(num_experts * ffn_dim, d_model, generator=g).bfloat16()
    out = dsd(blocks.cuda(), w.cuda(), dev, version=version)
    lay = build_layout(idx.numpy(), num_experts, ffn_dim, bs)
    assert out.shape == ((dev.row_offsets.numel() - 1) * bs, d_model)
    torch.testing.assert_close(out[: lay.num_rows].float().cpu(), oracle(blocks, w, lay), **TOL)
    if version in ZEROS_DEAD_ROWS:
        assert torch.all(out[lay.num_rows:] == 0)


def test_wide_tiles() -> None:
    # >= 1024 row blocks x 256-column slices: the 256-column tile path runs.
    lay = build_layout(routing_case("random", 65536, 8).numpy(), 8, 128, 128)
    assert lay.num_row_blocks >= 1024
    g = torch.Generator().manual_seed(4)
    blocks = (torch.randn(lay.col_indices.size, 128, 128, generator=g) / 12).bfloat16()
    w = torch.randn(8 * 128, 256, generator=g).bfloat16()
    torch.testing.assert_close(run(blocks, w, lay, 5).float().cpu(), oracle(blocks, w, lay), **TOL)


def test_long_rows() -> None:
    # 32 blocks per row block (K = 4096, the fine-grained shape's F).
    lay = build_layout(routing_case("zipf", 300, 4).numpy(), 4, 4096, 128)
    g = torch.Generator().manual_seed(5)
    blocks = (torch.randn(lay.col_indices.size, 128, 128, generator=g) / 64).bfloat16()
    w = torch.randn(4 * 4096, 256, generator=g).bfloat16()
    torch.testing.assert_close(run(blocks, w, lay, 5).float().cpu(), oracle(blocks, w, lay), **TOL)


BAD_INPUTS = {
    "fp32_weights": (lambda b, w: (b, w.float()), "bfloat16"),
    "fp16_blocks": (lambda b, w: (b.half(), w), "bfloat16"),
    "d_not_multiple": (lambda b, w: (b, w[:, :100].contiguous()), "multiple of 128"),
    "non_contiguous": (lambda b, w: (b, w.t().contiguous().t()), "contiguous"),
    "cpu_weights": (lambda b, w: (b, w.cpu()), "CUDA"),
}


@pytest.mark.parametrize("name", BAD_INPUTS)
def test_rejects_bad_input(name) -> None:
    lay, blocks, w = make_inputs("random", 20, 4, 128, 256, 64)
    change, match = BAD_INPUTS[name]
    b, w2 = change(blocks.cuda(), w.cuda())
    from sparsebench_amd import _C

    with pytest.raises(RuntimeError, match=match):
        _C.dsd_cuda(b, w2, torch.as_tensor(lay.row_offsets).cuda(), torch.as_tensor(lay.col_indices).cuda(), 1)


def test_rejects_unsupported_block_size_and_version() -> None:
    from sparsebench_amd import _C

    lay, blocks, w = make_inputs("random", 20, 4, 64, 256, 64)
    with pytest.raises(RuntimeError, match="unknown dsd version"):
        run(blocks, w, lay, 99)
    lay32 = build_layout(routing_case("random", 20, 4).numpy(), 4, 64, 32)
    blocks32 = torch.zeros(lay32.col_indices.size, 32, 32, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="64 or 128"):
        _C.dsd_cuda(blocks32, w.cuda(), torch.as_tensor(lay32.row_offsets).cuda(),
                    torch.as_tensor(lay32.col_indices).cuda(), 1)


def test_rejects_block_shape_mismatch() -> None:
    from sparsebench_amd.routing import build_topology_cuda
    from sparsebench_amd.spmm import dsd

    topo = build_topology_cuda(routing_case("random", 20, 4).cuda(), 4, 128, 64)
    blocks = torch.zeros(topo.nnz_blocks, 64, 64, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(4 * 128, 256, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="blocks must be"):
        dsd(blocks[:, :32], w, topo, 1)


@pytest.mark.parametrize(("bs", "d_model"), [(64, 256), (128, 128), (128, 384)])
def test_v5_rejects_shapes_it_does_not_support(bs, d_model) -> None:
    lay, blocks, w = make_inputs("random", 50, 4, 2 * bs, d_model, bs)
    with pytest.raises(RuntimeError, match="dsd v5 needs block size 128 and D a multiple of 256"):
        run(blocks, w, lay, 5)
