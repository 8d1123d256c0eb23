"""The layer on a routing given as assignments, and the GPU router (top-k,
token rounding fused with routing), against the CPU oracle.

The cases of the reference's tests/test_token_rounding.py:91-148, plus:
bit-exact router output (lists, weights, layout), the combine's list-order
summation on both token-grouping paths, the token-rounded layer without a
host sync under graph replay.

Tolerances: lists, layouts and the router's fp32 weights are exact (the
same fp32 operations in the same order); layer outputs use the reference's
assert_close(3e-2) and the north star's max rel err <= 2e-2 against fp32.
"""

import numpy as np
import pytest
import torch

from oracle.moe_ref import max_rel_err, moe_assigned_reference
from oracle.token_rounding_ref import keep_mask, token_rounding as token_rounding_ref, top_k_assignments as topk_ref
from oracle.topology_ref import device_layout
from sparsebench_amd.workloads import router_scores

pytestmark = pytest.mark.gpu

LAYER_TOL = {"rtol": 3e-2, "atol": 3e-2}


def make_layer(num_tokens, num_experts, d_model=256, ffn_dim=256, seed=0):
    # tests/test_token_rounding.py:101-106 (reference)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(num_tokens, d_model, generator=g).bfloat16().cuda()
    w1 = (torch.randn(num_experts, d_model, ffn_dim, generator=g) / d_model**0.5).bfloat16().cuda()
    w2 = (torch.randn(num_experts, ffn_dim, d_model, generator=g) / ffn_dim**0.5).bfloat16().cuda()
    return x, w1, w2


def tie_heavy_scores(num_tokens, num_experts, levels, seed):
    rng = np.random.default_rng(seed)
    return torch.from_numpy((rng.integers(0, levels, size=(num_tokens, num_experts)) / levels).astype(np.float32))


ROUTER_CASES = [  # (name, T, E, k, tile)
    ("uniform", 4096, 64, 2, 128), ("zipf", 4096, 64, 2, 128), ("uniform", 2000, 8, 2, 128),
    ("zipf", 3000, 16, 4, 128), ("uniform", 1000, 65, 3, 16), ("zipf", 777, 130, 2, 32),
    ("uniform", 50, 3, 1, 4), ("zipf", 16384, 128, 2, 128),
]


def scores_of(name, t, e, seed=0):
    if name.startswith("ties"):
        return tie_heavy_scores(t, e, int(name[4:]), seed)
    return router_scores(name, t, e, seed)


# ---------------------------------------------------------------- router ---

@pytest.mark.parametrize(("name", "t", "e", "k", "tile"), ROUTER_CASES + [("ties5", 300, 6, 2, 8),
                                                                       ("ties3", 129, 70, 2, 4)])
def test_top_k_assignments_exact(name, t, e, k, tile) -> None:
    from sparsebench_amd.token_rounding import top_k_assignments

    scores = scores_of(name, t, e)
    got = top_k_assignments(scores.cuda(), k)
    ref = topk_ref(scores.numpy(), k)
    assert torch.equal(got.token.cpu(), torch.from_numpy(ref.token))
    assert torch.equal(got.expert.cpu(), torch.from_numpy(ref.expert))
    assert torch.equal(got.weight.cpu(), torch.from_numpy(ref.weight))


@pytest.mark.parametrize("kernel", ["1", "2"])  # the top-k test hook: 1 = a wave per token, 2 = a lane per token
@pytest.mark.parametrize(("name", "t", "e", "k", "tile"), [("ties5", 300, 6, 2, 8), ("ties3", 129, 70, 2, 4),
                                                          ("uniform", 1000, 65, 3, 16), ("ties4", 700, 37, 5, 8),
                                                          ("zipf", 500, 1000, 16, 32), ("uniform", 333, 200, 9, 16)])
def test_both_top_k_forms_exact(kernel, name, t, e, k, tile, hooks) -> None:
    # The top-k kernel is chosen by E x k; each form, forced, must give the
    # oracle's list and the oracle's token rounding.
    from sparsebench_amd.token_rounding import token_rounding, top_k_assignments

    hooks.topk_kernel(kernel)
    scores = scores_of(name, t, e)
    got = top_k_assignments(scores.cuda(), k)
    ref = topk_ref(scores.numpy(), k)
    assert torch.equal(got.expert.cpu(), torch.from_numpy(ref.expert))
    assert torch.equal(got.weight.cpu(), torch.from_numpy(ref.weight))
    got = token_rounding(scores.cuda(), k, tile)
    ref = token_rounding_ref(scores.numpy(), k, tile)
    assert torch.equal(got.token.cpu(), torch.from_numpy(ref.token))
    assert torch.equal(got.expert.cpu(), torch.from_numpy(ref.expert))
    torch.testing.assert_close(got.weight.cpu(), torch.from_numpy(ref.weight), rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize(("name", "t", "e", "k", "tile"), ROUTER_CASES + [("ties5", 300, 6, 2, 8),
                                                                       ("ties3", 129, 70, 2, 4),
                                                                       ("ties1000", 64, 5, 2, 4)])
def test_token_rounding_exact(name, t, e, k, tile) -> None:
    from sparsebench_amd.token_rounding import token_rounding

    scores = scores_of(name, t, e)
    got = token_rounding(scores.cuda(), k, tile)
    ref = token_rounding_ref(scores.numpy(), k, tile)
    assert torch.equal(got.token.cpu(), torch.from_numpy(ref.token))
    assert torch.equal(got.expert.cpu(), torch.from_numpy(ref.expert))
    # A token whose kept scores are all 0 gets 0/0 on both sides.
    torch.testing.assert_close(got.weight.cpu(), torch.from_numpy(ref.weight), rtol=0, atol=0, equal_nan=True)


def test_token_rounding_hand_worked_case() -> None:
    # tests/test_token_rounding.py:19-33 (reference)
    from sparsebench_amd.token_rounding import token_rounding

    s0 = torch.tensor([0.9, 0.8, 0.7, 0.6, 0.55, 0.1, 0.2, 0.3])
    a = token_rounding(torch.stack([s0, 1 - s0], dim=1).cuda(), k=1, tile=4)
    kept = set(zip(a.token.tolist(), a.expert.tolist()))
    assert {t for t, e in kept if e == 0} == {0, 1, 2, 3}
    assert {t for t, e in kept if e == 1} == {4, 5, 6, 7}
    assert torch.allclose(a.weight.cpu(), torch.ones(8))


def expected_assigned_layout(token, expert, num_tokens, num_experts, ffn_dim, bs):
    """device_layout of the list as [N, 1], row_token mapped from copy to token."""
    token = np.asarray(token)
    lay = device_layout(np.asarray(expert).reshape(-1, 1), num_experts, ffn_dim, bs)
    rt = lay.row_token.astype(np.int64)
    mapped = np.where(rt >= 0, token[np.clip(rt, 0, None)], -1).astype(np.int32)
    return lay, mapped


def assert_prefix_then(buf: torch.Tensor, ref: np.ndarray, fill: int) -> None:
    """buf starts with ref and is `fill` after it (buffers sized for more)."""
    b = buf.cpu().numpy()
    assert np.array_equal(b[: ref.size], ref)
    assert np.all(b[ref.size:] == fill)


@pytest.mark.parametrize(("name", "t", "e", "k", "tile"), [("uniform", 4096, 64, 2, 128), ("zipf", 2000, 8, 2, 128),
                                                          ("uniform", 1000, 65, 3, 16)])
def test_fused_routing_layout(name, t, e, k, tile) -> None:
    from sparsebench_amd.routing import route_rounded

    ffn_dim, bs = 512, 128
    scores = scores_of(name, t, e)
    r = route_rounded(scores.cuda(), k, ffn_dim, bs, tile)
    ref = token_rounding_ref(scores.numpy(), k, tile)
    n = ref.token.size
    assert int(r.num_assignments) == n
    assert_prefix_then(r.token_of_copy, ref.token.astype(np.int32), -1)
    assert_prefix_then(r.expert_of_copy, ref.expert.astype(np.int32), -1)
    lay, row_token = expected_assigned_layout(ref.token, ref.expert, t, e, ffn_dim, bs)
    topo = r.topology
    assert np.array_equal(topo.tokens_per_expert.cpu().numpy(), lay.tokens_per_expert)
    assert np.array_equal(topo.padded_offsets.cpu().numpy(), lay.padded_offsets)
    assert_prefix_then(topo.copy_row, lay.copy_row, -1)
    nrows = int(lay.padded_offsets[-1])
    assert_prefix_then(topo.row_token, row_token[:nrows], -1)
    nrb = nrows // bs
    assert_prefix_then(topo.row_block_expert, lay.row_block_expert[:nrb], -1)
    assert_prefix_then(topo.row_offsets, lay.row_offsets[: nrb + 1], nrb * (ffn_dim // bs))
    assert_prefix_then(topo.col_indices, lay.col_indices[: nrb * (ffn_dim // bs)], -1)
    assert int(topo.error) == 0
    offs = np.zeros(t + 1, dtype=np.int64)
    np.add.at(offs, ref.token + 1, 1)
    assert np.array_equal(r.token_offsets.cpu().numpy(), np.cumsum(offs))


def test_token_rounding_keeps_tile_multiples_without_padding() -> None:
    from sparsebench_amd.routing import route_rounded

    scores = router_scores("zipf", 4096, 64)
    r = route_rounded(scores.cuda(), 2, 512, 128, 128)
    keep, target = keep_mask(scores.numpy(), 2, 128)
    assert np.array_equal(r.topology.tokens_per_expert.cpu().numpy(), target)
    assert int(r.topology.padded_offsets[-1]) == int(target.sum())  # no padding row at all


# ------------------------------------------------------------ token CSR ---

@pytest.mark.parametrize("order", ["sorted", "shuffled", "reversed"])
@pytest.mark.parametrize(("num_tokens", "n"), [(1, 5), (100, 1), (700, 3000), (5000, 9000), (20000, 40000)])
def test_token_csr(order, num_tokens, n) -> None:
    from sparsebench_amd import _C

    rng = np.random.default_rng(n)
    token = np.sort(rng.integers(0, num_tokens, size=n))
    if order == "shuffled":
        rng.shuffle(token)
    elif order == "reversed":
        token = token[::-1].copy()
    routed = rng.random(n) > 0.1  # some copies were not routed
    copy_row = np.where(routed, np.arange(n), -1).astype(np.int32)
    offs, copies = _C.token_csr_cuda(torch.from_numpy(token).cuda(), torch.from_numpy(copy_row).cuda(), num_tokens)
    listed = np.nonzero(routed)[0]
    exp_copies = listed[np.argsort(token[listed], kind="stable")]
    counts = np.bincount(token[listed], minlength=num_tokens)
    assert np.array_equal(offs.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    assert_prefix_then(copies, exp_copies.astype(np.int32), -1)


# ------------------------------------------------------------ the layer ---

@pytest.mark.parametrize("name", ["uniform", "zipf"])
def test_moe_assigned_with_token_rounding(name) -> None:
    # tests/test_token_rounding.py:109-120 (reference)
    from sparsebench_amd.moe import moe_forward_assigned
    from sparsebench_amd.token_rounding import token_rounding

    num_tokens, num_experts = 2048, 16
    x, w1, w2 = make_layer(num_tokens, num_experts)
    a = token_rounding(router_scores(name, num_tokens, num_experts).cuda(), 2)
    out = moe_forward_assigned(x, a.token, a.expert, a.weight, w1, w2)
    ref = moe_assigned_reference(x, a.token, a.expert, a.weight, w1, w2)
    torch.testing.assert_close(out.float().cpu(), ref, **LAYER_TOL)
    assert max_rel_err(out.float().cpu(), ref) <= 2e-2


def test_moe_assigned_handles_0_and_3_experts_per_token() -> None:
    # tests/test_token_rounding.py:122-134 (reference)
    from sparsebench_amd.moe import moe_forward_assigned

    x, w1, w2 = make_layer(6, 4)
    token = torch.tensor([1, 2, 2, 2, 3, 3, 4, 4, 5, 5], device="cuda")
    expert = torch.tensor([0, 1, 2, 3, 0, 1, 2, 3, 0, 3], device="cuda")
    weight = torch.rand(10, generator=torch.Generator().manual_seed(1)).cuda()
    out = moe_forward_assigned(x, token, expert, weight, w1, w2)
    ref = moe_assigned_reference(x, token, expert, weight, w1, w2)
    torch.testing.assert_close(out.float().cpu(), ref, **LAYER_TOL)
    assert torch.all(out[0] == 0)


def test_moe_assigned_equals_moe_forward_for_plain_top_k() -> None:
    # tests/test_token_rounding.py:137-148 (reference). Here the two paths sum
    # the same products in the same order, so they agree bit for bit.
    from sparsebench_amd.moe import moe_forward, moe_forward_assigned
    from sparsebench_amd.token_rounding import top_k_assignments

    num_tokens, num_experts = 1000, 8
    x, w1, w2 = make_layer(num_tokens, num_experts)
    scores = router_scores("zipf", num_tokens, num_experts).cuda()
    top_s, top_i = scores.topk(2, dim=1)
    weight = (top_s / top_s.sum(1, keepdim=True)).bfloat16()
    a = top_k_assignments(scores, 2)
    assert torch.equal(a.expert.view(num_tokens, 2), top_i)
    expected = moe_forward(x, top_i, weight, w1, w2)
    got = moe_forward_assigned(x, a.token, a.expert, weight.reshape(-1), w1, w2)
    assert torch.equal(got, expected)


@pytest.mark.parametrize("dtypes", [(torch.int64, torch.int64), (torch.int32, torch.int32), (torch.int32, torch.int64)])
def test_moe_assigned_list_order(dtypes) -> None:
    # A token's copies are summed in list order (as the reference's
    # index_add_ does on the CPU). Moving whole tokens around, with each
    # token's copies kept in order, takes the unsorted path of the token
    # grouping and must give the same bits; any other permutation gives the
    # same values to rounding.
    from sparsebench_amd.moe import moe_forward_assigned
    from sparsebench_amd.token_rounding import token_rounding

    num_tokens, num_experts = 1500, 16
    x, w1, w2 = make_layer(num_tokens, num_experts, seed=3)
    a = token_rounding(router_scores("zipf", num_tokens, num_experts, seed=3).cuda(), 2, 64)
    base = moe_forward_assigned(x, a.token, a.expert, a.weight, w1, w2)
    assert torch.equal(base, moe_forward_assigned(x, a.token, a.expert, a.weight, w1, w2))  # deterministic
    token_perm = torch.randperm(num_tokens, generator=torch.Generator().manual_seed(0)).cuda()
    moved = torch.sort(token_perm[a.token], stable=True).indices  # tokens reordered, copies kept in order
    got = moe_forward_assigned(x, a.token[moved].to(dtypes[0]), a.expert[moved].to(dtypes[1]), a.weight[moved],
                               w1, w2)
    assert torch.equal(got, base)
    perm = torch.randperm(a.token.numel(), generator=torch.Generator().manual_seed(1)).cuda()
    shuffled = moe_forward_assigned(x, a.token[perm].to(dtypes[0]), a.expert[perm].to(dtypes[1]), a.weight[perm],
                                    w1, w2)
    torch.testing.assert_close(shuffled.float(), base.float(), rtol=1e-2, atol=1e-2)


def test_moe_assigned_empty_list() -> None:
    from sparsebench_amd.moe import moe_forward_assigned

    x, w1, w2 = make_layer(10, 4)
    empty = torch.empty(0, dtype=torch.int64, device="cuda")
    out = moe_forward_assigned(x, empty, empty, torch.empty(0, device="cuda"), w1, w2)
    assert torch.equal(out, torch.zeros_like(x))


def test_moe_assigned_bad_ids_are_skipped_and_flagged() -> None:
    from sparsebench_amd.moe import moe_forward_assigned
    from sparsebench_amd.routing import route_assigned

    x, w1, w2 = make_layer(8, 4)
    token = torch.tensor([0, 1, 9, 2, 3, -1, 4], device="cuda")  # 9 and -1: not tokens
    expert = torch.tensor([0, 1, 2, 7, 3, 1, 2], device="cuda")  # 7: not an expert
    weight = torch.ones(7, device="cuda")
    r = route_assigned(token, expert, 8, 4, 256, 128)
    assert int(r.topology.error) == 1
    assert r.topology.copy_row.cpu().tolist()[2:4] == [-1, -1] and int(r.topology.copy_row[5]) == -1
    out = moe_forward_assigned(x, token, expert, weight, w1, w2)
    ok = torch.tensor([0, 1, 4, 6])
    ref = moe_assigned_reference(x, token.cpu()[ok], expert.cpu()[ok], weight.cpu()[ok], w1, w2)
    torch.testing.assert_close(out.float().cpu(), ref, **LAYER_TOL)


def test_assigned_routing_layout_exact() -> None:
    from sparsebench_amd.routing import route_assigned

    rng = np.random.default_rng(5)
    n, t, e, ffn_dim, bs = 3000, 1000, 12, 512, 128
    token = rng.integers(0, t, size=n)
    expert = rng.integers(0, e, size=n)
    r = route_assigned(torch.from_numpy(token).cuda(), torch.from_numpy(expert).cuda(), t, e, ffn_dim, bs)
    lay, row_token = expected_assigned_layout(token, expert, t, e, ffn_dim, bs)
    topo = r.topology
    for name in ["tokens_per_expert", "padded_offsets", "copy_row", "row_block_expert", "row_offsets",
                 "col_indices"]:
        assert np.array_equal(getattr(topo, name).cpu().numpy(), getattr(lay, name)), name
    assert np.array_equal(topo.row_token.cpu().numpy(), row_token)


# ---------------------------------------- token rounding fused, no sync ---

def test_moe_forward_rounded_equals_two_step_form() -> None:
    from sparsebench_amd.moe import moe_forward_assigned, moe_forward_rounded
    from sparsebench_amd.token_rounding import token_rounding

    num_tokens, num_experts = 4096, 64
    x, w1, w2 = make_layer(num_tokens, num_experts, 512, 512, seed=7)
    scores = router_scores("uniform", num_tokens, num_experts, seed=7).cuda()
    fused = moe_forward_rounded(x, scores, 2, w1, w2)
    a = token_rounding(scores, 2)
    assert torch.equal(fused, moe_forward_assigned(x, a.token, a.expert, a.weight, w1, w2))
    ref = moe_assigned_reference(x, a.token, a.expert, a.weight, w1, w2)
    assert max_rel_err(fused.float().cpu(), ref) <= 2e-2


def test_moe_forward_rounded_graph_replay() -> None:
    # Captured once; each replay takes new scores and x written in place, with
    # no host sync inside (the layout and list length stay on the GPU).
    from sparsebench_amd.moe import moe_forward_rounded

    num_tokens, num_experts = 2048, 32
    x, w1, w2 = make_layer(num_tokens, num_experts, seed=11)
    scores = router_scores("zipf", num_tokens, num_experts, seed=11).cuda()
    moe_forward_rounded(x, scores, 2, w1, w2)  # warm up outside the graph
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = moe_forward_rounded(x, scores, 2, w1, w2)
    for seed in (1, 2, 3):
        new_x, _, _ = make_layer(num_tokens, num_experts, seed=100 + seed)
        x.copy_(new_x)
        scores.copy_(router_scores("zipf" if seed % 2 else "uniform", num_tokens, num_experts, seed=seed).cuda())
        graph.replay()
        torch.cuda.synchronize()
        eager = moe_forward_rounded(x, scores, 2, w1, w2)
        assert torch.equal(out, eager)
