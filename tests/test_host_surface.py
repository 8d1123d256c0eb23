"""Host-side surface on the CPU: the drop-in module aliasing of INTEGRATION.md,
the reference-shaped dataclasses, and argument errors raised before any GPU call."""

import dataclasses
import sys

import pytest
import torch


def test_reference_import_path_works_unchanged() -> None:
    # The reference's own imports (sparsebench/moe.py:15-16, tests/test_moe.py,
    # tests/test_token_rounding.py), with no sys.modules set-up by the caller.
    from sparsebench import _C as c
    from sparsebench.moe import moe_forward, moe_forward_assigned  # noqa: F401
    from sparsebench.routing import DeviceTopology, build_topology_cuda, route_device  # noqa: F401
    from sparsebench.spmm import dsd, sdd  # noqa: F401
    from sparsebench.token_rounding import (  # noqa: F401
        Assignments, round_counts, routing_change, token_rounding, top_k_assignments)
    from sparsebench.topology import Topology  # noqa: F401
    from sparsebench.workloads import router_scores, routing_case  # noqa: F401

    import sparsebench
    import sparsebench_amd.moe

    assert {"arch_probe", "build_topology_cuda", "sdd_cuda", "dsd_cuda"} <= set(dir(c))
    # One module object under both names: patching one patches the other.
    assert sparsebench.moe is sparsebench_amd.moe
    assert sys.modules["sparsebench._C"] is c


def test_topology_fields_match_the_reference_order() -> None:
    from sparsebench_amd.routing import DeviceTopology
    from sparsebench_amd.topology import Topology

    common = ["block_size", "num_experts", "ffn_blocks", "tokens_per_expert", "padded_offsets", "row_token",
              "copy_row", "row_block_expert", "row_offsets", "col_indices"]
    assert [f.name for f in dataclasses.fields(Topology)] == common
    assert [f.name for f in dataclasses.fields(DeviceTopology)] == common + ["error"]


def test_build_topology_rejects_cpu_tensor() -> None:
    from sparsebench_amd.routing import build_topology_cuda

    with pytest.raises(RuntimeError, match="CUDA"):
        build_topology_cuda(torch.tensor([[0, 1]]), 8, 32, 16)


def test_dsd_rejects_cpu_weights() -> None:
    from sparsebench_amd import _C

    with pytest.raises(RuntimeError, match="CUDA"):
        _C.dsd_cuda(torch.zeros(1, 64, 64, dtype=torch.bfloat16), torch.zeros(64, 128, dtype=torch.bfloat16),
                    torch.zeros(2, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), 1)


def test_sdd_wrapper_rejects_block_size_64_before_the_gpu() -> None:
    from sparsebench_amd.spmm import sdd
    from sparsebench_amd.topology import Topology

    z = torch.zeros(1, dtype=torch.int32)
    topo = Topology(64, 4, 4, z, z, z, z, z, z, z)
    with pytest.raises(ValueError, match="block size 128"):
        sdd(torch.zeros(2, 64, dtype=torch.bfloat16), torch.zeros(4, 64, 256, dtype=torch.bfloat16), topo)


def test_moe_forward_rejects_mismatched_shapes_before_the_gpu() -> None:
    from sparsebench_amd.moe import moe_forward

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w1 = torch.zeros(2, 64, 256, dtype=torch.bfloat16)
    idx = torch.zeros(4, 2, dtype=torch.long)
    with pytest.raises(ValueError, match="w2"):
        moe_forward(x, idx, torch.ones(4, 2), w1, torch.zeros(2, 64, 256, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="x must be"):
        moe_forward(x, idx, torch.ones(4, 1), w1, torch.zeros(2, 256, 64, dtype=torch.bfloat16))


def test_workload_shapes_and_flops() -> None:
    from sparsebench_amd.workloads import SHAPES, routing_case

    fg = SHAPES["fine_grained"]
    assert fg.useful_flops == 2 * 2 * 4096 * 2 * 1024 * 4096  # 137.44 GFLOP, as the reference counts it
    idx = routing_case("zipf_perm", 4096, 64, seed=0)
    assert idx.shape == (4096, 2) and bool((idx[:, 0] != idx[:, 1]).all())
    assert torch.equal(idx, routing_case("zipf_perm", 4096, 64, seed=0))
    # Zipf over a permutation: the hottest expert is not expert 0 for this seed, and counts are skewed.
    counts = torch.bincount(idx.flatten(), minlength=64)
    assert int(counts.max()) > 4 * int(counts.float().median())


def test_assignments_fields_match_the_reference() -> None:
    from sparsebench_amd.token_rounding import Assignments

    assert [f.name for f in dataclasses.fields(Assignments)] == ["token", "expert", "weight"]


def test_round_counts_nearest_ties_down() -> None:
    # tests/test_token_rounding.py:13-16 (reference): host arithmetic on a few counts
    from sparsebench_amd.token_rounding import round_counts

    counts = torch.tensor([0, 1, 63, 64, 65, 128, 191, 192, 200])
    expected = torch.tensor([0, 0, 0, 0, 128, 128, 128, 128, 256])
    assert torch.equal(round_counts(counts, 128, 10_000), expected)


def test_router_scores_match_the_reference_recipe() -> None:
    from sparsebench_amd.workloads import router_scores

    s = router_scores("zipf", 100, 8)
    assert s.shape == (100, 8) and s.dtype == torch.float32
    torch.testing.assert_close(s.sum(dim=1), torch.ones(100))
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(100, 8, generator=g) - 1.2 * torch.log(torch.arange(1, 9, dtype=torch.float32))
    assert torch.equal(s, torch.softmax(logits, dim=-1))
    with pytest.raises(ValueError):
        router_scores("skewed", 4, 4)


def test_moe_forward_assigned_rejects_bad_lists_before_the_gpu() -> None:
    from sparsebench_amd.moe import moe_forward_assigned

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w1 = torch.zeros(2, 64, 256, dtype=torch.bfloat16)
    w2 = torch.zeros(2, 256, 64, dtype=torch.bfloat16)
    t = torch.zeros(3, dtype=torch.long)
    with pytest.raises(ValueError, match="one entry per copy"):
        moe_forward_assigned(x, t, t, torch.ones(2), w1, w2)
    with pytest.raises(ValueError, match="w2"):
        moe_forward_assigned(x, t, t, torch.ones(3), w1, w1)
    # An empty list is answered on the host, like the reference (moe.py:77-78).
    e = torch.zeros(0, dtype=torch.long)
    assert torch.equal(moe_forward_assigned(x, e, e, torch.ones(0), w1, w2), torch.zeros_like(x))


def test_router_rejects_cpu_scores() -> None:
    from sparsebench_amd.token_rounding import token_rounding, top_k_assignments

    with pytest.raises(RuntimeError, match="CUDA"):
        token_rounding(torch.rand(10, 4), 2)
    with pytest.raises(RuntimeError, match="CUDA"):
        top_k_assignments(torch.rand(10, 4), 2)


def test_reference_support_modules_are_not_provided() -> None:
    # The import path covers the forward path only; the reference's benchmark
    # and test support modules are absent, as INTEGRATION.md states.
    import importlib

    import sparsebench.topology

    for name in ("sparsebench.reference", "sparsebench.timing", "sparsebench.baselines"):
        with pytest.raises(ImportError):
            importlib.import_module(name)
    for fn in ("build_topology", "bsr_to_dense", "dense_to_bsr"):
        assert not hasattr(sparsebench.topology, fn)
