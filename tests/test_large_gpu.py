"""Full-size checks against the fp32 oracle: the benchmark's largest shapes,
and an activation tensor x of more than 2 GiB.

The layer at the Mixtral-like shape (K = 14336 in the DSD: 448 K steps of
32) and at config 5's shape (T = 16384, E = 128, F = 768) runs at its real
size; the oracle then recomputes a seeded subset of tokens, each with its
own routing and gates and the full weights (oracle/moe_ref.py's fp32 loop
over experts). Gates: max |out - ref| / max |ref| <= 2e-2 and the
reference's assert_close(rtol=3e-2, atol=3e-2) (tests/test_moe.py:18-34).

x over 2 GiB: the reference indexes x in 64 bits (csrc/sdd.cu:71-72) and
accepts any x (sdd.cu:151-153). At T = 264192, D = 4096 and at T = 528384,
D = 2048 with F = 512 and 768 (x = 2.16 GB, one shape per SDD tile form) the
SDD gathers rows past the 2 GiB mark; sampled H rows, including every row of
the highest token ids, are checked against GELU(x[token] @ W1[e]) in fp64.
"""

import pytest
import torch

from oracle.moe_ref import gelu_erf, layer_reference_fp32, max_rel_err
from sparsebench_amd.workloads import SHAPES, LayerShape, make_layer

pytestmark = pytest.mark.gpu

REL = 2e-2


def check_token_subset(out, x, idx, gates, w1, w2, num: int, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    sel = torch.randperm(x.shape[0], generator=g)[:num].sort().values.to(x.device)
    expected = layer_reference_fp32(x[sel], idx[sel], gates[sel], w1, w2)
    got = out[sel]
    assert max_rel_err(got, expected) <= REL
    torch.testing.assert_close(got.float().cpu(), expected, rtol=3e-2, atol=3e-2)


@pytest.mark.parametrize("name, routing, num", [("mixtral", "random", 384), ("replay_sweep", "zipf_perm", 512)])
def test_benchmark_shape_against_oracle(name: str, routing: str, num: int) -> None:
    from sparsebench_amd.moe import moe_forward

    shape = SHAPES[name]
    x, idx, gates, w1, w2 = make_layer(shape, routing, seed=0)
    out = moe_forward(x, idx, gates, w1, w2)
    torch.cuda.synchronize()
    check_token_subset(out, x, idx, gates, w1, w2, num, seed=11)


WIDE = LayerShape("wide_x", 264192, 4096, 512, 8)
# x over 2 GiB in each of sb_sdd's three tile forms (sdd_tile_for): the
# deep 128 x 512 tile (D >= 4096), the wide one (D < 4096, F % 512 == 0) and
# the narrow 128 x 256 tile (F % 512 != 0), each gathering x with 64-bit
# addresses.
WIDE_FORMS = {
    "deep": WIDE,
    "wide": LayerShape("wide_x_d2048", 528384, 2048, 512, 8),
    "narrow": LayerShape("wide_x_f768", 528384, 2048, 768, 8),
}


def wide_inputs(shape: LayerShape = WIDE):
    x, idx, gates, w1, w2 = make_layer(shape, "random", seed=3)
    assert x.numel() * x.element_size() > 2**31
    return x, idx, gates, w1, w2


def sampled_rows(row_token: torch.Tensor, num_rows: int, num_tokens: int) -> torch.Tensor:
    """Padded rows to check: every row of the 64 highest token ids, random
    real rows, and some padding rows."""
    g = torch.Generator().manual_seed(5)
    real = torch.nonzero(row_token[:num_rows] >= 0).flatten()
    top = torch.nonzero(row_token[:num_rows] >= num_tokens - 64).flatten()
    pad = torch.nonzero(row_token[:num_rows] < 0).flatten()
    rnd = real[torch.randperm(real.numel(), generator=g)[:192]]
    return torch.cat([top, rnd, pad[:16]]).unique()


@pytest.mark.parametrize(("entry", "form"), [("sdd_cuda", "deep"), ("sdd_experts_cuda", "deep"),
                                             ("sdd_experts_cuda", "wide"), ("sdd_experts_cuda", "narrow")])
def test_sdd_accepts_x_over_2gib(entry: str, form: str) -> None:
    from sparsebench_amd import _C
    from sparsebench_amd.routing import route_device
    from sparsebench_amd.spmm import sdd

    shape = WIDE_FORMS[form]
    x, idx, _, w1, _ = wide_inputs(shape)
    e, f = shape.num_experts, shape.ffn_dim
    topo = route_device(idx, e, f, 128)
    h = sdd(x, w1, topo) if entry == "sdd_cuda" else _C.sdd_experts_cuda(x, w1, topo, True)
    torch.cuda.synchronize()
    row_token = topo.row_token.cpu()
    rbe = topo.row_block_expert.cpu()
    num_rows = int(topo.padded_offsets[-1])
    rows = sampled_rows(row_token, num_rows, shape.num_tokens)
    assert (row_token[rows] >= shape.num_tokens - 64).sum() >= 64  # rows past the 2 GiB mark are in the sample
    fb = f // 128
    w1_cpu = w1.double().cpu()
    for r in rows.tolist():
        rb, i = divmod(r, 128)
        got = h[rb * fb:(rb + 1) * fb, i, :].reshape(f).float().cpu()
        tok = int(row_token[r])
        if tok < 0:
            assert torch.all(got == 0), f"padding row {r} must be zero"
            continue
        want = gelu_erf(x[tok].double().cpu() @ w1_cpu[int(rbe[rb])]).float()
        torch.testing.assert_close(got, want, rtol=1.6e-2, atol=1.6e-2, msg=f"row {r} token {tok}")


def test_layer_with_x_over_2gib() -> None:
    from sparsebench_amd.moe import moe_forward

    x, idx, gates, w1, w2 = wide_inputs()
    out = moe_forward(x, idx, gates, w1, w2)
    torch.cuda.synchronize()
    check_token_subset(out, x, idx, gates, w1, w2, 256, seed=13)
    top = torch.arange(WIDE.num_tokens - 64, WIDE.num_tokens, device=x.device)
    expected = layer_reference_fp32(x[top], idx[top], gates[top], w1, w2)
    assert max_rel_err(out[top], expected) <= REL
