"""The combine kernel against the closed form (fp32 products summed over k).

The kernel rounds one fp32 sum per element to bf16, like the oracle does
after its fp32 sum, so the two agree to one bf16 rounding step plus fp32
summation order: rtol 1e-2, atol 1e-5.
"""

import numpy as np
import pytest
import torch

from oracle.moe_ref import combine_reference

pytestmark = pytest.mark.gpu

TOL = {"rtol": 1e-2, "atol": 1e-5}


def make(num_tokens: int, k: int, d_model: int, rows: int, gate_dtype, seed: int = 0, skipped: float = 0.0):
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(rows, d_model, generator=g).bfloat16()
    copy_row = torch.randperm(rows, generator=g)[: num_tokens * k].int()
    if skipped:
        drop = torch.rand(num_tokens * k, generator=g) < skipped
        copy_row[drop] = -1
    w = torch.rand(num_tokens, k, generator=g).to(gate_dtype)
    return y, copy_row, w


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("num_tokens", "k", "d_model"),
                         [(1, 1, 8), (300, 2, 256), (77, 4, 1024), (4096, 2, 1024), (50, 3, 64), (33, 8, 128)])
def test_matches_closed_form(gate_dtype, num_tokens, k, d_model) -> None:
    from sparsebench_amd.moe import combine

    y, copy_row, w = make(num_tokens, k, d_model, num_tokens * k + 37, gate_dtype)
    out = combine(y.cuda(), copy_row.cuda(), w.cuda())
    assert out.dtype == torch.bfloat16 and out.shape == (num_tokens, d_model)
    torch.testing.assert_close(out.float().cpu(), combine_reference(y, copy_row.numpy(), w), **TOL)


def test_skipped_copies_add_nothing() -> None:
    from sparsebench_amd.moe import combine

    y, copy_row, w = make(500, 2, 128, 1100, torch.float32, skipped=0.3)
    out = combine(y.cuda(), copy_row.cuda(), w.cuda())
    torch.testing.assert_close(out.float().cpu(), combine_reference(y, copy_row.numpy(), w), **TOL)
    both = (copy_row.view(500, 2) < 0).all(dim=1)
    assert torch.all(out.cpu()[both] == 0)


def test_exact_on_representable_values() -> None:
    # Gates of 1 and 0.5 and small integer-valued rows: every product and sum
    # is exact in fp32 and representable in bf16, so the result is bit-exact.
    from sparsebench_amd.moe import combine

    y = torch.arange(-64, 64, dtype=torch.float32).repeat(6, 1).bfloat16()  # [6, 128]
    copy_row = torch.tensor([5, 0, 1, 4, 2, 3], dtype=torch.int32)
    w = torch.tensor([[1.0, 0.5], [0.5, 0.5], [1.0, 1.0]])
    out = combine(y.cuda(), copy_row.cuda(), w.cuda()).float().cpu()
    expected = combine_reference(y, copy_row.numpy(), w)
    assert torch.equal(out, expected)


def test_valid_tokens_stops_at_the_device_count() -> None:
    from sparsebench_amd import _C

    y, copy_row, w = make(64, 2, 64, 200, torch.float32)
    vt = torch.tensor([40], dtype=torch.int32, device="cuda")
    out = _C.combine_cuda(y.cuda(), copy_row.cuda(), w.cuda(), vt)
    torch.testing.assert_close(out[:40].float().cpu(), combine_reference(y, copy_row.numpy(), w)[:40], **TOL)
    full = _C.combine_cuda(y.cuda(), copy_row.cuda(), w.cuda())
    assert torch.equal(out[:40], full[:40])


@pytest.mark.parametrize("k", [1, 2, 3, 4, 8])
def test_sums_in_slot_order_exactly(k) -> None:
    # out = bf16(((0 + y0*g0) + y1*g1) + ...), fp32 throughout, skipped
    # copies adding nothing: a sequential fp32 sum gives the same bits.
    from sparsebench_amd.moe import combine

    num_tokens, d_model = 200, 64
    y, copy_row, w = make(num_tokens, k, d_model, num_tokens * k + 5, torch.float32, skipped=0.2)
    out = combine(y.cuda(), copy_row.cuda(), w.cuda()).cpu()
    yf = y.float().numpy()
    rows = copy_row.numpy().reshape(num_tokens, k)
    wf = w.float().numpy()
    acc = np.zeros((num_tokens, d_model), dtype=np.float32)
    for j in range(k):
        r = rows[:, j]
        ok = r >= 0
        acc[ok] = (acc[ok] + yf[r[ok]] * wf[ok, j][:, None]).astype(np.float32)
    assert torch.equal(out, torch.from_numpy(acc).bfloat16())


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("k", [1, 2])
def test_bit_exact_to_reference_arithmetic(gate_dtype, k) -> None:
    # With at most two products the reference's .sum() has one order, so
    # rounded products then one fp32 add must give the oracle's bits exactly.
    from sparsebench_amd.moe import combine

    y, copy_row, w = make(1000, k, 512, 1000 * k + 9, gate_dtype, seed=4, skipped=0.1)
    out = combine(y.cuda(), copy_row.cuda(), w.cuda()).cpu()
    assert torch.equal(out, combine_reference(y, copy_row.numpy(), w).bfloat16())


@pytest.mark.parametrize(("num_tokens", "d_model"), [(5000, 24), (701, 1000), (333, 1032), (90, 2040), (70001, 8)])
def test_any_row_width_bit_exact(num_tokens, d_model) -> None:
    # Row widths of 3, 125, 129, 255 and 1 16-byte chunks: each lane splits
    # its flat number into token and chunk, which must give every lane its
    # own (token, chunk) at any width.
    from sparsebench_amd import _C
    from sparsebench_amd.moe import combine

    y, copy_row, w = make(num_tokens, 2, d_model, num_tokens * 2 + 3, torch.float32, seed=d_model, skipped=0.05)
    want = combine_reference(y, copy_row.numpy(), w).bfloat16()
    out = combine(y.cuda(), copy_row.cuda(), w.cuda()).cpu()
    assert torch.equal(out, want)
    # The assigned combine, with each token's copies listed in slot order.
    offsets = torch.arange(0, 2 * num_tokens + 1, 2, dtype=torch.int32)
    out_a = _C.combine_assigned_cuda(y.cuda(), copy_row.cuda(), w.reshape(-1).cuda(), offsets.cuda(), None,
                                     num_tokens).cpu()
    assert torch.equal(out_a, want)
