"""DSD with the combine fused into its epilogue against the two-kernel path.

The fused kernel sums each token's rows in slot order with the same fp32
operations as the combine kernel, so the outputs must be identical bit for
bit, on every call (the arrival counters are reused across calls), for
every routing case, gate dtype, a token count limited on the device, and
under graph replay.
"""

import pytest
import torch

from oracle.moe_ref import layer_reference_fp32, max_rel_err
from sparsebench_amd.workloads import routing_case

pytestmark = pytest.mark.gpu


def make(num_tokens, num_experts, d_model, ffn_dim, case, seed=0, k=2, gate_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(num_tokens, d_model, generator=g).bfloat16().cuda()
    w1 = (torch.randn(num_experts, d_model, ffn_dim, generator=g) / d_model**0.5).bfloat16().cuda()
    w2 = (torch.randn(num_experts, ffn_dim, d_model, generator=g) / ffn_dim**0.5).bfloat16().cuda()
    idx = routing_case(case, num_tokens, num_experts, seed, k).cuda()
    gates = torch.softmax(torch.randn(num_tokens, idx.shape[1], generator=g), -1).to(gate_dtype).cuda()
    return x, idx, gates, w1, w2


@pytest.mark.parametrize("case", ["random", "zipf", "skewed", "empty_middle", "two_experts_only"])
@pytest.mark.parametrize(("num_tokens", "num_experts", "d_model", "ffn_dim"),
                         [(700, 16, 256, 512), (4096, 64, 1024, 512), (1000, 8, 2048, 256), (333, 4, 512, 256)])
def test_fused_equals_two_kernels(case, num_tokens, num_experts, d_model, ffn_dim) -> None:
    from sparsebench_amd.moe import moe_forward

    x, idx, gates, w1, w2 = make(num_tokens, num_experts, d_model, ffn_dim, case)
    ref = moe_forward(x, idx, gates, w1, w2)
    for _ in range(3):  # counters left at zero by every call
        assert torch.equal(moe_forward(x, idx, gates, w1, w2, fused_combine=True), ref)


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_gate_dtypes_and_fp32_parity(gate_dtype) -> None:
    from sparsebench_amd.moe import moe_forward

    x, idx, gates, w1, w2 = make(512, 8, 256, 512, "random", seed=3, k=4, gate_dtype=gate_dtype)
    out = moe_forward(x, idx, gates, w1, w2, fused_combine=True)
    assert torch.equal(out, moe_forward(x, idx, gates, w1, w2))
    ref = layer_reference_fp32(x.cpu(), idx.cpu(), gates.cpu(), w1.cpu(), w2.cpu())
    assert max_rel_err(out.float().cpu(), ref) <= 2e-2


def test_fused_skips_bad_ids_and_zeroes_orphan_tokens() -> None:
    from sparsebench_amd.moe import moe_forward

    x, idx, gates, w1, w2 = make(300, 8, 256, 256, "random", seed=5)
    idx[5] = torch.tensor([8, -1])  # token 5: both copies bad -> zero row
    idx[9, 1] = 99                  # token 9: one copy skipped
    out = moe_forward(x, idx, gates, w1, w2, fused_combine=True)
    assert torch.equal(out, moe_forward(x, idx, gates, w1, w2))
    assert torch.all(out[5] == 0)


def test_fused_valid_tokens_and_graph_replay() -> None:
    from sparsebench_amd.moe import moe_forward

    t_max = 2048
    x, idx, gates, w1, w2 = make(t_max, 32, 512, 512, "zipf", seed=7)
    valid = torch.tensor([t_max], dtype=torch.int32, device="cuda")
    moe_forward(x, idx, gates, w1, w2, valid_tokens=valid, fused_combine=True)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = moe_forward(x, idx, gates, w1, w2, valid_tokens=valid, fused_combine=True)
    for seed, t in ((1, 2048), (2, 700), (3, 1500), (4, 2048)):
        nx, nidx, ngates, _, _ = make(t_max, 32, 512, 512, "random" if seed % 2 else "zipf", seed=seed)
        x.copy_(nx)
        idx.copy_(nidx)
        gates.copy_(ngates)
        valid.fill_(t)
        graph.replay()
        torch.cuda.synchronize()
        ref = moe_forward(x, idx, gates, w1, w2, valid_tokens=valid)
        assert torch.equal(out[:t], ref[:t])


@pytest.mark.parametrize("variant", [25, 32, 58, 62, 63, 64])
def test_fused_every_tile_form(variant, monkeypatch) -> None:
    from sparsebench_amd.moe import moe_forward

    x, idx, gates, w1, w2 = make(1500, 16, 1024, 512, "zipf", seed=11)
    ref = moe_forward(x, idx, gates, w1, w2)
    monkeypatch.setenv("SPARSEBENCH_DSD_VARIANT", str(variant))
    assert torch.equal(moe_forward(x, idx, gates, w1, w2, fused_combine=True), ref)
    assert torch.equal(moe_forward(x, idx, gates, w1, w2, fused_combine=True), ref)
