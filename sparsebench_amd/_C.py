"""The operator surface of the reference's pybind11 module `sparsebench._C`
(csrc/bindings.cpp:5-16, csrc/ops.hpp:11-36), over the gfx950 C ABI.

Same four functions, same keyword names, same outputs, and the same
RuntimeError messages for bad arguments (the checks of csrc/routing.cu:198-224,
csrc/sdd.cu:126-153, csrc/dsd.cpp:29-61, csrc/dsd_v5.cu:108-110,
csrc/smoke.cu:24), in the same order. Outputs come from torch's caching
allocator on the input's device and all work is enqueued on torch's current
stream, so nothing here syncs and every call can be captured in a graph.

combine_cuda is this build's addition: the combine step of moe_forward as one
kernel.
"""

from __future__ import annotations

import ctypes

import torch

from sparsebench_amd._lib import check, lib, stream_of

_I32_MAX = 2**31 - 1
_MAX_EXPERTS = 1024
_DSD_TILE_N = 128
# dsd version code -> dead row blocks written as zeros (versions 1-3) or left unwritten (4 on)
_DSD_VERSIONS = {1: True, 2: True, 21: True, 3: True, 31: True, 4: False, 41: False, 5: False}
_GATE_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _fail(msg: str) -> None:
    raise RuntimeError(msg)


def _shape(t: torch.Tensor) -> str:
    return "[" + ", ".join(str(s) for s in t.shape) + "]"


def _check_index(t: torch.Tensor, name: str) -> None:
    if not (t.is_cuda and t.dtype == torch.int32 and t.dim() == 1 and t.is_contiguous()):
        _fail(f"{name} must be a contiguous 1-D int32 CUDA tensor")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_TEST_HOOKS = {"expert_gate": 0, "topk_kernel": 1}


def set_test_hook(name: str, value: int) -> None:
    """Forces one of the library's own choices for tests (include/sparsebench_hip.h:
    expert_gate 1 = expert tiles, 2 = row blocks; topk_kernel 1 = wave form,
    2 = lane form); 0 restores the choice."""
    if name not in _TEST_HOOKS:
        raise ValueError(f"unknown test hook {name!r}")
    check(lib().sb_set_test_hook(_TEST_HOOKS[name], int(value)))


def arch_probe(n: int) -> torch.Tensor:
    """int32[n] filled with the architecture number of the code that ran (950 on gfx950)."""
    if n <= 0:
        _fail(f"arch_probe: n must be positive, got {n}")
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    check(lib().sb_arch_probe(out.data_ptr(), n, stream_of(out.device)))
    return out


def routing_sizes(num_copies: int, num_experts: int, ffn_dim: int, block_size: int) -> tuple[int, int, int]:
    """(max_row_blocks, max_rows, workspace int32 elements) for n = T*k copies."""
    rb, rows, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    check(lib().sb_routing_sizes(num_copies, num_experts, ffn_dim, block_size,
                                 ctypes.byref(rb), ctypes.byref(rows), ctypes.byref(ws)))
    return rb.value, rows.value, ws.value


def build_topology_cuda(
    expert_idx: torch.Tensor,
    num_experts: int,
    ffn_dim: int,
    block_size: int,
    valid_tokens: torch.Tensor | None = None,
) -> list[torch.Tensor]:
    """Routing -> block-sparse layout on the GPU, no host sync.

    Returns, in order: tokens_per_expert [E], padded_offsets [E+1],
    row_token [max_rows], copy_row [T*k], row_block_expert [max_row_blocks],
    row_offsets [max_row_blocks+1], col_indices [max_row_blocks*ffn_blocks],
    error [1] (all int32; csrc/ops.hpp:13-21).

    valid_tokens (this build's extension, default None = reference behaviour):
    an int32 CUDA scalar T' <= T; copies of tokens >= T' are ignored.
    """
    if not expert_idx.is_cuda:
        _fail("expert_idx must be a CUDA tensor")
    if expert_idx.dim() != 2 or expert_idx.shape[0] == 0 or expert_idx.shape[1] == 0:
        _fail(f"expert_idx must be [T, k] with T, k > 0, got {_shape(expert_idx)}")
    if expert_idx.dtype not in (torch.int32, torch.int64):
        _fail(f"expert_idx must be int32 or int64, got {expert_idx.dtype}")
    if not expert_idx.is_contiguous():
        _fail("expert_idx must be contiguous")
    if not 0 < num_experts <= _MAX_EXPERTS:
        _fail(f"num_experts must be in [1, {_MAX_EXPERTS}], got {num_experts}")
    if not 0 < block_size <= _I32_MAX:
        _fail("block_size must be in [1, 2^31)")
    if ffn_dim <= 0 or ffn_dim % block_size != 0:
        _fail(f"ffn_dim ({ffn_dim}) must be a positive multiple of block_size ({block_size})")
    num_tokens, k = expert_idx.shape
    n = num_tokens * k
    # Worst case: every expert wastes block_size - 1 rows (csrc/routing.cu:213-224).
    max_row_blocks = (n + num_experts * (block_size - 1)) // block_size
    max_rows = max_row_blocks * block_size
    ffn_blocks = ffn_dim // block_size
    if max_rows > _I32_MAX // ffn_dim or max_row_blocks * ffn_blocks >= _I32_MAX or n > _I32_MAX:
        _fail("problem too large for int32 indexing")
    if valid_tokens is not None:
        if not (valid_tokens.is_cuda and valid_tokens.dtype == torch.int32 and valid_tokens.numel() == 1):
            _fail("valid_tokens must be a one-element int32 CUDA tensor")

    dev = expert_idx.device
    opts = {"dtype": torch.int32, "device": dev}
    num_chunks = (n + 1023) // 1024
    workspace = torch.empty(num_chunks * (num_experts + 1), **opts)
    tokens_per_expert = torch.empty(num_experts, **opts)
    padded_offsets = torch.empty(num_experts + 1, **opts)
    row_token = torch.empty(max_rows, **opts)
    copy_row = torch.empty(n, **opts)
    row_block_expert = torch.empty(max_row_blocks, **opts)
    row_offsets = torch.empty(max_row_blocks + 1, **opts)
    col_indices = torch.empty(max_row_blocks * ffn_blocks, **opts)
    error = torch.empty(1, **opts)
    check(lib().sb_routing(
        expert_idx.data_ptr(), 1 if expert_idx.dtype == torch.int64 else 0, num_tokens, k, num_experts, ffn_dim,
        block_size, _ptr(valid_tokens), workspace.data_ptr(), tokens_per_expert.data_ptr(),
        padded_offsets.data_ptr(), row_token.data_ptr(), copy_row.data_ptr(), row_block_expert.data_ptr(),
        row_offsets.data_ptr(), col_indices.data_ptr(), error.data_ptr(), stream_of(dev),
    ))
    return [tokens_per_expert, padded_offsets, row_token, copy_row, row_block_expert, row_offsets, col_indices, error]


def sdd_cuda(
    x: torch.Tensor,
    w1: torch.Tensor,
    row_token: torch.Tensor,
    row_block_expert: torch.Tensor,
    row_offsets: torch.Tensor,
    num_nnz: int,
    apply_gelu: bool,
) -> torch.Tensor:
    """H blocks [num_nnz, 128, 128] bf16 = (gelu)(x[row_token] @ w1[expert]) on the layout's blocks."""
    if not (x.is_cuda and w1.is_cuda and x.device == w1.device):
        _fail("x and w1 must be on the same GPU")
    if x.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16:
        _fail("x and w1 must be bfloat16")
    if not (x.is_contiguous() and w1.is_contiguous()):
        _fail("x and w1 must be contiguous")
    if not (x.dim() == 2 and w1.dim() == 3 and w1.shape[1] == x.shape[1]):
        _fail(f"x must be [T, D] and w1 [E, D, F], got {_shape(x)} and {_shape(w1)}")
    _check_index(row_token, "row_token")
    _check_index(row_block_expert, "row_block_expert")
    _check_index(row_offsets, "row_offsets")
    if x.data_ptr() % 16 or w1.data_ptr() % 16:
        _fail("x and w1 must be 16-byte aligned")
    d_model, ffn_dim = x.shape[1], w1.shape[2]
    num_row_blocks = row_offsets.numel() - 1
    if d_model <= 0 or d_model % 64:
        _fail(f"sdd needs D ({d_model}) to be a multiple of 64")
    if ffn_dim <= 0 or ffn_dim % 256:
        _fail(f"sdd needs F ({ffn_dim}) to be a multiple of 256")
    if row_token.numel() != num_row_blocks * 128:
        _fail(f"sdd needs block size 128: row_token has {row_token.numel()} rows for {num_row_blocks} row blocks")
    if row_block_expert.numel() != num_row_blocks:
        _fail("row_block_expert must have one entry per row block")
    if num_nnz != num_row_blocks * (ffn_dim // 128):
        _fail(f"expected {num_row_blocks * (ffn_dim // 128)} blocks (row blocks x F/128), got {num_nnz}")
    if num_row_blocks * (ffn_dim // 256) > _I32_MAX or ffn_dim * d_model > _I32_MAX:
        _fail("problem too large")
    out = torch.empty(num_nnz, 128, 128, dtype=w1.dtype, device=w1.device)
    if num_row_blocks <= 0:
        return out
    check(lib().sb_sdd(
        x.data_ptr(), w1.data_ptr(), row_token.data_ptr(), row_block_expert.data_ptr(), row_offsets.data_ptr(),
        out.data_ptr(), x.shape[0], d_model, ffn_dim, w1.shape[0], num_row_blocks, 1 if apply_gelu else 0,
        stream_of(x.device),
    ))
    return out


def dsd_cuda(
    blocks: torch.Tensor, w: torch.Tensor, row_offsets: torch.Tensor, col_indices: torch.Tensor, version: int
) -> torch.Tensor:
    """out [(len(row_offsets)-1)*bs, D] bf16 = BSR(blocks, row_offsets, col_indices) @ w.

    Every version code of the reference is accepted and gives the same
    results; codes 1, 2, 21, 3, 31 write dead row blocks as zeros, codes 4,
    41, 5 leave them unwritten, and 5 needs block size 128 and D % 256 == 0.
    """
    if not (blocks.is_cuda and w.is_cuda):
        _fail("blocks and w must be CUDA tensors")
    if not (blocks.device == w.device and row_offsets.device == w.device and col_indices.device == w.device):
        _fail("all inputs must be on the same GPU")
    if blocks.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        _fail("blocks and w must be bfloat16")
    if not (blocks.is_contiguous() and w.is_contiguous()):
        _fail("blocks and w must be contiguous")
    if not (blocks.dim() == 3 and blocks.shape[1] == blocks.shape[2]):
        _fail(f"blocks must be [nnz, bs, bs], got {_shape(blocks)}")
    if w.dim() != 2:
        _fail(f"w must be [E*F, D], got {_shape(w)}")
    _check_index(row_offsets, "row_offsets")
    _check_index(col_indices, "col_indices")
    bs, d_model = blocks.shape[1], w.shape[1]
    num_row_blocks = row_offsets.numel() - 1
    if bs not in (64, 128):
        _fail(f"block size must be 64 or 128, got {bs}")
    if d_model <= 0 or d_model % _DSD_TILE_N:
        _fail(f"D ({d_model}) must be a positive multiple of {_DSD_TILE_N}")
    if d_model // _DSD_TILE_N > 65535:
        _fail("D too large for grid y")
    if w.shape[0] % bs:
        _fail(f"w rows ({w.shape[0]}) must be a multiple of the block size ({bs})")
    if num_row_blocks < 0:
        _fail("row_offsets must have at least one entry")
    if blocks.shape[0] != col_indices.numel():
        _fail(f"blocks has {blocks.shape[0]} blocks but col_indices has {col_indices.numel()}")
    if num_row_blocks * bs > _I32_MAX:
        _fail("too many row blocks")
    if num_row_blocks * (d_model // _DSD_TILE_N) > _I32_MAX:
        _fail("too many tiles for a 1-D grid")
    if blocks.data_ptr() % 16:
        _fail("blocks must be 16-byte aligned")
    if w.data_ptr() % 16:
        _fail("w must be 16-byte aligned")
    out = torch.empty(num_row_blocks * bs, d_model, dtype=w.dtype, device=w.device)
    if num_row_blocks == 0:
        return out
    if version not in _DSD_VERSIONS:
        _fail(f"unknown dsd version {version}")
    if version == 5 and (bs != 128 or d_model % 256):
        _fail(f"dsd v5 needs block size 128 and D a multiple of 256, got block size {bs}, D {d_model}")
    check(lib().sb_dsd(
        blocks.data_ptr(), w.data_ptr(), row_offsets.data_ptr(), col_indices.data_ptr(), out.data_ptr(),
        blocks.shape[0], w.shape[0], num_row_blocks, bs, d_model, 1 if _DSD_VERSIONS[version] else 0,
        stream_of(w.device),
    ))
    return out


def _check_expert_layout(topo, device: torch.device) -> None:
    if topo.block_size != 128:
        _fail(f"expert tiles need block size 128, got {topo.block_size}")
    for name in ("tokens_per_expert", "padded_offsets", "row_token", "row_block_expert", "row_offsets", "col_indices"):
        t = getattr(topo, name)
        _check_index(t, name)
        if t.device != device:
            _fail("all inputs must be on the same GPU")
    if topo.padded_offsets.numel() != topo.num_experts + 1 or topo.tokens_per_expert.numel() != topo.num_experts:
        _fail("tokens_per_expert / padded_offsets do not match the expert count")
    max_row_blocks = topo.row_token.numel() // 128
    if (topo.row_token.numel() != max_row_blocks * 128 or topo.row_block_expert.numel() != max_row_blocks
            or topo.row_offsets.numel() != max_row_blocks + 1
            or topo.col_indices.numel() != max_row_blocks * topo.ffn_blocks):
        _fail("the routing layout's arrays do not have worst-case sizes of one layout")


def sdd_experts_cuda(x: torch.Tensor, w1: torch.Tensor, topo, apply_gelu: bool) -> torch.Tensor:
    """SDD of the MoE layer (this build's addition): expert-major tiles when
    the routing is balanced, else row-block tiles, chosen on the GPU; for
    F % 512 != 0, each expert's row blocks in pairs (every row written).

    topo: a routing layout from route_device / route_assigned / route_rounded.
    Returns H blocks [max_row_blocks*F/128, 128, 128] bf16 whose real rows are
    bit-identical to sdd_cuda's; padding rows past each expert's last 32-row
    group may be left unwritten (the layer never reads them).
    """
    if not (x.is_cuda and w1.is_cuda and x.device == w1.device):
        _fail("x and w1 must be on the same GPU")
    if x.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16:
        _fail("x and w1 must be bfloat16")
    if not (x.is_contiguous() and w1.is_contiguous()):
        _fail("x and w1 must be contiguous")
    if not (x.dim() == 2 and w1.dim() == 3 and w1.shape[1] == x.shape[1]):
        _fail(f"x must be [T, D] and w1 [E, D, F], got {_shape(x)} and {_shape(w1)}")
    _check_expert_layout(topo, x.device)
    num_experts, d_model, ffn_dim = w1.shape
    if num_experts != topo.num_experts or ffn_dim != topo.ffn_blocks * 128:
        _fail("w1 does not match the routing layout")
    max_row_blocks = topo.row_token.numel() // 128
    out = torch.empty(max_row_blocks * (ffn_dim // 128), 128, 128, dtype=w1.dtype, device=w1.device)
    check(lib().sb_sdd_experts(
        x.data_ptr(), w1.data_ptr(), topo.row_token.data_ptr(), topo.row_block_expert.data_ptr(),
        topo.row_offsets.data_ptr(), topo.tokens_per_expert.data_ptr(), topo.padded_offsets.data_ptr(),
        out.data_ptr(), x.shape[0], d_model, ffn_dim, num_experts, max_row_blocks, 1 if apply_gelu else 0,
        stream_of(x.device),
    ))
    return out


def dsd_experts_cuda(h: torch.Tensor, w2_cat: torch.Tensor, topo) -> torch.Tensor:
    """DSD (version 5) of the MoE layer (this build's addition): expert-major
    tiles when the routing is balanced, else the per-row-block kernel, chosen
    on the GPU.

    h: sdd_experts_cuda's (or sdd_cuda's) blocks on topo's layout; w2_cat
    [E*F, D]. Returns y [max_row_blocks*128, D] bf16 whose real rows are
    bit-identical to dsd_cuda's; padding rows may be left unwritten.
    """
    if not (h.is_cuda and w2_cat.is_cuda and h.device == w2_cat.device):
        _fail("h and w must be on the same GPU")
    if h.dtype != torch.bfloat16 or w2_cat.dtype != torch.bfloat16:
        _fail("h and w must be bfloat16")
    if not (h.is_contiguous() and w2_cat.is_contiguous()):
        _fail("h and w must be contiguous")
    _check_expert_layout(topo, h.device)
    max_row_blocks = topo.row_token.numel() // 128
    ffn_dim = topo.ffn_blocks * 128
    if h.dim() != 3 or h.shape != (max_row_blocks * topo.ffn_blocks, 128, 128):
        _fail(f"h must be [{max_row_blocks * topo.ffn_blocks}, 128, 128] for this layout, got {_shape(h)}")
    if w2_cat.dim() != 2 or w2_cat.shape[0] != topo.num_experts * ffn_dim:
        _fail(f"w must be [E*F, D] = [{topo.num_experts * ffn_dim}, D], got {_shape(w2_cat)}")
    d_model = w2_cat.shape[1]
    out = torch.empty(max_row_blocks * 128, d_model, dtype=w2_cat.dtype, device=w2_cat.device)
    check(lib().sb_dsd_experts(
        h.data_ptr(), w2_cat.data_ptr(), topo.tokens_per_expert.data_ptr(), topo.padded_offsets.data_ptr(),
        topo.row_block_expert.data_ptr(), topo.row_offsets.data_ptr(), topo.col_indices.data_ptr(), out.data_ptr(),
        max_row_blocks, topo.num_experts, topo.copy_row.numel(), ffn_dim, d_model, stream_of(h.device),
    ))
    return out


def expert_tiles_fit(d_model: int, ffn_dim: int, max_row_blocks: int) -> bool:
    """Whether sdd_experts_cuda / dsd_experts_cuda take this shape (else the per-row-block kernels)."""
    h_bytes = max_row_blocks * (ffn_dim // 128) * 128 * 128 * 2
    return (d_model % 256 == 0 and ffn_dim % 256 == 0 and h_bytes < 2**31 and ffn_dim * d_model * 2 < 2**31)


def combine_cuda(
    y: torch.Tensor,
    copy_row: torch.Tensor,
    expert_weight: torch.Tensor,
    valid_tokens: torch.Tensor | None = None,
) -> torch.Tensor:
    """out [T, D] bf16: each token's k rows of y, gate-weighted, summed in fp32.

    y [rows, D] bf16, copy_row [T*k] int32 (row of copy t*k+j, -1 = skipped),
    expert_weight [T, k] bf16/fp16/fp32. Rows t >= valid_tokens (if given) are
    left unwritten.
    """
    if not (y.is_cuda and copy_row.is_cuda and expert_weight.is_cuda):
        _fail("y, copy_row and expert_weight must be CUDA tensors")
    if y.dtype != torch.bfloat16 or y.dim() != 2 or not y.is_contiguous():
        _fail(f"y must be a contiguous [rows, D] bfloat16 tensor, got {_shape(y)} {y.dtype}")
    _check_index(copy_row, "copy_row")
    if expert_weight.dim() != 2 or expert_weight.numel() != copy_row.numel():
        _fail(f"expert_weight must be [T, k] with T*k == len(copy_row), got {_shape(expert_weight)}")
    gates = expert_weight if expert_weight.dtype in _GATE_DTYPES else expert_weight.float()
    gates = gates.contiguous()
    num_tokens, k = expert_weight.shape
    out = torch.empty(num_tokens, y.shape[1], dtype=y.dtype, device=y.device)
    if num_tokens == 0:
        return out
    check(lib().sb_combine(
        y.data_ptr(), copy_row.data_ptr(), gates.data_ptr(), _GATE_DTYPES[gates.dtype], out.data_ptr(),
        num_tokens, k, y.shape[1], y.shape[0], _ptr(valid_tokens), stream_of(y.device),
    ))
    return out


# ---- routing given as assignments; router (this build's C ABI, no pybind11
# counterpart in the reference: there these steps are torch code in
# sparsebench/moe.py:59-91 and sparsebench/token_rounding.py) ----


def _check_copy_list(t: torch.Tensor, name: str) -> None:
    if not (t.is_cuda and t.dim() == 1 and t.dtype in (torch.int32, torch.int64) and t.is_contiguous()):
        _fail(f"{name} must be a contiguous 1-D int32 or int64 CUDA tensor")


def build_topology_assigned_cuda(
    token_of_copy: torch.Tensor,
    expert_of_copy: torch.Tensor,
    num_tokens: int,
    num_experts: int,
    ffn_dim: int,
    block_size: int,
    valid_tokens: torch.Tensor | None = None,
) -> list[torch.Tensor]:
    """The routing of a flat list (copy c: token_of_copy[c] -> expert_of_copy[c]),
    as build_topology_cuda with k = 1 and row_token holding token ids.
    Same 8 outputs, sized for N = len(list). No host sync."""
    _check_copy_list(token_of_copy, "token_of_copy")
    _check_copy_list(expert_of_copy, "expert_of_copy")
    n = expert_of_copy.numel()
    if token_of_copy.numel() != n or n == 0:
        _fail("token_of_copy and expert_of_copy must be non-empty and of the same length")
    if token_of_copy.device != expert_of_copy.device:
        _fail("token_of_copy and expert_of_copy must be on the same GPU")
    if not 0 < num_tokens <= _I32_MAX:
        _fail(f"num_tokens must be in [1, 2^31), got {num_tokens}")
    if valid_tokens is not None:
        if not (valid_tokens.is_cuda and valid_tokens.dtype == torch.int32 and valid_tokens.numel() == 1):
            _fail("valid_tokens must be a one-element int32 CUDA tensor")
    max_row_blocks, max_rows, ws = routing_sizes(n, num_experts, ffn_dim, block_size)
    dev = expert_of_copy.device
    opts = {"dtype": torch.int32, "device": dev}
    workspace = torch.empty(ws, **opts)
    outs = [torch.empty(num_experts, **opts), torch.empty(num_experts + 1, **opts), torch.empty(max_rows, **opts),
            torch.empty(n, **opts), torch.empty(max_row_blocks, **opts), torch.empty(max_row_blocks + 1, **opts),
            torch.empty(max_row_blocks * (ffn_dim // block_size), **opts), torch.empty(1, **opts)]
    check(lib().sb_routing_assigned(
        expert_of_copy.data_ptr(), 1 if expert_of_copy.dtype == torch.int64 else 0, token_of_copy.data_ptr(),
        1 if token_of_copy.dtype == torch.int64 else 0, n, num_tokens, num_experts, ffn_dim, block_size,
        _ptr(valid_tokens), workspace.data_ptr(), *(o.data_ptr() for o in outs), stream_of(dev),
    ))
    return outs


def token_csr_cuda(token_of_copy: torch.Tensor, copy_row: torch.Tensor, num_tokens: int
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """(token_offsets [T+1], token_copies [N]): each token's routed copies in
    ascending copy order. Deterministic, no host sync."""
    _check_copy_list(token_of_copy, "token_of_copy")
    _check_index(copy_row, "copy_row")
    n = token_of_copy.numel()
    if copy_row.numel() != n or n == 0:
        _fail("copy_row must have one entry per copy")
    dev = token_of_copy.device
    offsets = torch.empty(num_tokens + 1, dtype=torch.int32, device=dev)
    copies = torch.empty(n, dtype=torch.int32, device=dev)
    check(lib().sb_token_csr(token_of_copy.data_ptr(), 1 if token_of_copy.dtype == torch.int64 else 0,
                             copy_row.data_ptr(), n, num_tokens, offsets.data_ptr(), copies.data_ptr(),
                             stream_of(dev)))
    return offsets, copies


def combine_assigned_cuda(
    y: torch.Tensor,
    copy_row: torch.Tensor,
    weight_of_copy: torch.Tensor,
    token_offsets: torch.Tensor,
    token_copies: torch.Tensor | None,
    num_tokens: int,
    valid_tokens: torch.Tensor | None = None,
) -> torch.Tensor:
    """out [T, D] bf16: out[t] = sum over t's copies c (token_copies[token_offsets[t]:
    token_offsets[t+1]], or c = the index itself when token_copies is None) of
    fp32(y[copy_row[c]]) * fp32(weight_of_copy[c]), fp32 sum in copy order; 0 for
    a token with no copy."""
    if not (y.is_cuda and copy_row.is_cuda and weight_of_copy.is_cuda):
        _fail("y, copy_row and weight_of_copy must be CUDA tensors")
    if y.dtype != torch.bfloat16 or y.dim() != 2 or not y.is_contiguous():
        _fail(f"y must be a contiguous [rows, D] bfloat16 tensor, got {_shape(y)} {y.dtype}")
    _check_index(copy_row, "copy_row")
    _check_index(token_offsets, "token_offsets")
    if token_copies is not None:
        _check_index(token_copies, "token_copies")
    if token_offsets.numel() != num_tokens + 1:
        _fail(f"token_offsets must have T+1 = {num_tokens + 1} entries, got {token_offsets.numel()}")
    if weight_of_copy.dim() != 1 or weight_of_copy.numel() < copy_row.numel():
        _fail("weight_of_copy must be 1-D with one entry per copy")
    weights = weight_of_copy if weight_of_copy.dtype in _GATE_DTYPES else weight_of_copy.float()
    weights = weights.contiguous()
    out = torch.empty(num_tokens, y.shape[1], dtype=y.dtype, device=y.device)
    if num_tokens == 0:
        return out
    check(lib().sb_combine_assigned(
        y.data_ptr(), copy_row.data_ptr(), weights.data_ptr(), _GATE_DTYPES[weights.dtype], token_offsets.data_ptr(),
        _ptr(token_copies), out.data_ptr(), num_tokens, y.shape[1], y.shape[0], _ptr(valid_tokens),
        stream_of(y.device),
    ))
    return out


def _check_scores(scores: torch.Tensor) -> None:
    if not (scores.is_cuda and scores.dtype == torch.float32 and scores.dim() == 2 and scores.is_contiguous()):
        _fail("scores must be a contiguous [T, E] float32 CUDA tensor")
    if scores.shape[0] == 0 or scores.shape[1] == 0:
        _fail(f"scores must be [T, E] with T, E > 0, got {_shape(scores)}")


def router_topk_cuda(scores: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(top_idx [T, k] int32, top_weight [T, k] fp32): the k best experts of each
    token, best first (equal scores: lower expert first), and the picked
    scores over their sum."""
    _check_scores(scores)
    num_tokens, num_experts = scores.shape
    idx = torch.empty(num_tokens, k, dtype=torch.int32, device=scores.device)
    weight = torch.empty(num_tokens, k, dtype=torch.float32, device=scores.device)
    check(lib().sb_router_topk(scores.data_ptr(), num_tokens, num_experts, k, idx.data_ptr(), weight.data_ptr(),
                               stream_of(scores.device)))
    return idx, weight


def router_sizes(num_tokens: int, num_experts: int, k: int, tile: int, block_size: int, ffn_dim: int
                 ) -> tuple[int, int, int, int]:
    """(list capacity, max_row_blocks, max_rows, workspace int32 elements) of token rounding."""
    cap, rb, rows, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    check(lib().sb_router_sizes(num_tokens, num_experts, k, tile, block_size, ffn_dim, ctypes.byref(cap),
                                ctypes.byref(rb), ctypes.byref(rows), ctypes.byref(ws)))
    return cap.value, rb.value, rows.value, ws.value


def token_rounding_cuda(scores: torch.Tensor, k: int, tile: int, ffn_dim: int, block_size: int
                        ) -> dict[str, torch.Tensor]:
    """Token rounding fused with routing, no host sync. Returns the list
    (token_of_copy / expert_of_copy int32, weight_of_copy fp32, capacity-sized,
    -1 / -1 / 0 past the end), num_assignments [1], token_offsets [T+1], and the
    8 routing outputs of build_topology_assigned_cuda for that list."""
    _check_scores(scores)
    num_tokens, num_experts = scores.shape
    cap, max_row_blocks, max_rows, ws = router_sizes(num_tokens, num_experts, k, tile, block_size, ffn_dim)
    dev = scores.device
    i32 = {"dtype": torch.int32, "device": dev}
    out = {
        "token_of_copy": torch.empty(cap, **i32),
        "expert_of_copy": torch.empty(cap, **i32),
        "weight_of_copy": torch.empty(cap, dtype=torch.float32, device=dev),
        "num_assignments": torch.empty(1, **i32),
        "token_offsets": torch.empty(num_tokens + 1, **i32),
        "tokens_per_expert": torch.empty(num_experts, **i32),
        "padded_offsets": torch.empty(num_experts + 1, **i32),
        "row_token": torch.empty(max_rows, **i32),
        "copy_row": torch.empty(cap, **i32),
        "row_block_expert": torch.empty(max_row_blocks, **i32),
        "row_offsets": torch.empty(max_row_blocks + 1, **i32),
        "col_indices": torch.empty(max_row_blocks * (ffn_dim // block_size), **i32),
        "error": torch.empty(1, **i32),
    }
    workspace = torch.empty(ws, **i32)
    check(lib().sb_token_rounding(
        scores.data_ptr(), num_tokens, num_experts, k, tile, block_size, ffn_dim, workspace.data_ptr(),
        *(t.data_ptr() for t in out.values()), stream_of(dev),
    ))
    return out
