"""Seeded synthetic inputs: routing patterns and whole MoE layers.

The routing patterns are the reference's test cases (sparsebench/workloads.py:
12-36 there), drawn with the same torch generator calls so that a seed gives
the same expert_idx as the reference's tests: each one is a case that breaks
kernels (empty experts, one overloaded expert, Zipf skew). `zipf_perm` is the
benchmark variant: Zipf popularity over a seeded permutation of the experts.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

ZIPF_EXPONENT = 1.2
CASE_NAMES = ["random", "skewed", "two_experts_only", "empty_middle", "zipf"]


def _zipf_weights(num_experts: int) -> torch.Tensor:
    rank = torch.arange(1, num_experts + 1, dtype=torch.float64)
    return rank.pow(-ZIPF_EXPONENT)


def routing_case(name: str, num_tokens: int, num_experts: int, seed: int = 0, k: int = 2) -> torch.Tensor:
    """expert_idx [T, k] int64 on the CPU; k distinct experts per token (k = 2 except for random / zipf*)."""
    g = torch.Generator().manual_seed(seed)
    if name == "random":  # uniform: the k largest of E uniform draws
        return torch.rand(num_tokens, num_experts, generator=g).topk(k, dim=-1).indices
    if name == "skewed":  # every first choice is expert 0, the second spreads over the rest
        second = torch.randint(1, num_experts, (num_tokens,), generator=g)
        return torch.stack((torch.zeros_like(second), second), dim=1)
    if name == "two_experts_only":  # all other experts get nothing
        return torch.tensor([[0, 1]]).expand(num_tokens, 2).contiguous()
    if name == "empty_middle":  # experts 1 .. E-2 get nothing
        pair = torch.tensor([[0, num_experts - 1]]).expand(num_tokens, 2)
        return pair[:, torch.randperm(2, generator=g)].contiguous()
    if name == "zipf":  # expert e drawn with weight 1/(e+1)^1.2, without replacement
        w = _zipf_weights(num_experts).expand(num_tokens, -1)
        return torch.multinomial(w, k, replacement=False, generator=g)
    if name == "zipf_perm":  # Zipf popularity over a seeded random ranking of the experts
        ranking = torch.randperm(num_experts, generator=g)
        w = torch.empty(num_experts, dtype=torch.float64)
        w[ranking] = _zipf_weights(num_experts)
        return torch.multinomial(w.expand(num_tokens, -1), k, replacement=False, generator=g)
    raise ValueError(name)


def router_scores(name: str, num_tokens: int, num_experts: int, seed: int = 0) -> torch.Tensor:
    """Softmax router scores [T, E] fp32 on the CPU, for routers that need full
    scores (token rounding), drawn with the same generator calls as the
    reference (sparsebench/workloads.py:39-52): "uniform" = N(0, 1) logits;
    "zipf" adds -1.2 log(rank) per expert, so popularity falls off like
    routing_case("zipf")."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(num_tokens, num_experts, generator=g)
    if name == "zipf":
        logits = logits - ZIPF_EXPONENT * torch.log(torch.arange(1, num_experts + 1, dtype=torch.float32))
    elif name != "uniform":
        raise ValueError(name)
    return torch.softmax(logits, dim=-1)


def softmax_gates(num_tokens: int, k: int, seed: int, device: str | torch.device = "cpu") -> torch.Tensor:
    """[T, k] gate weights: softmax over the k picks of N(0, 1) logits (fp32)."""
    g = torch.Generator().manual_seed(seed)
    return torch.softmax(torch.randn(num_tokens, k, generator=g), dim=-1).to(device)


@dataclass(frozen=True)
class LayerShape:
    name: str
    num_tokens: int
    d_model: int
    ffn_dim: int
    num_experts: int
    top_k: int = 2

    @property
    def useful_flops(self) -> int:
        """2 matmuls x 2 FLOP per MAC x T*k rows x D x F (no padding)."""
        return 2 * 2 * self.num_tokens * self.top_k * self.d_model * self.ffn_dim


# The configurations of the benchmark (T, D, F, E).
SHAPES = {
    "cpu_reference": LayerShape("cpu_reference", 256, 128, 512, 8),
    "fine_grained": LayerShape("fine_grained", 4096, 1024, 4096, 64),
    "mixtral": LayerShape("mixtral", 4096, 4096, 14336, 8),
    "replay_sweep": LayerShape("replay_sweep", 16384, 2048, 768, 128),
}


def make_layer(
    shape: LayerShape,
    routing: str = "random",
    seed: int = 0,
    device: str | torch.device = "cuda",
    dtype: torch.dtype = torch.bfloat16,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(x [T, D], expert_idx [T, k] int64, gates [T, k] fp32, w1 [E, D, F], w2 [E, F, D]).

    x ~ N(0, 1); W1 ~ N(0, 1/D) and W2 ~ N(0, 1/F) so activations stay about
    N(0, 1). Tensors are drawn on `device` with a generator of that device
    (large layers never pass through host memory).
    """
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    t, d, f, e = shape.num_tokens, shape.d_model, shape.ffn_dim, shape.num_experts
    x = torch.randn(t, d, generator=g, device=device, dtype=torch.float32).to(dtype)
    w1 = torch.empty(e, d, f, device=device, dtype=dtype)
    w2 = torch.empty(e, f, d, device=device, dtype=dtype)
    for i in range(e):  # one expert at a time: no fp32 copy of all weights
        w1[i] = (torch.randn(d, f, generator=g, device=device) / math.sqrt(d)).to(dtype)
        w2[i] = (torch.randn(f, d, generator=g, device=device) / math.sqrt(f)).to(dtype)
    idx = routing_case(routing, t, e, seed, shape.top_k).to(device)
    gates = softmax_gates(t, shape.top_k, seed + 1, device)
    return x, idx, gates, w1, w2
