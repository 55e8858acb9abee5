"""Attention-state merges on gfx950 against the CPU oracle (oracle/merge.py).

The extreme-LSE table, the in-place and NaN-payload cases and the strided
partial stacks are data from flash_attn_mps tests/test_merge.py (cited per
case).  Checks: fp32 outputs within 1e-6 of the fp64 oracle, 16-bit outputs
within one rounding of it, LSE within 1e-6, sentinels untouched.
"""
import pytest
import torch

from flash_attn_mps_amd._merge import merge_attn_states, merge_partials
from harness import max_err
from oracle import merge as omerge

pytestmark = pytest.mark.gpu

INF = float("inf")

# Pairs of LSE values that stress the weights: +-1000, one side -inf, both
# -inf, far apart (test_merge.py:14-15).
LEFT_LSE = [[1000.0, -1000.0, -INF], [-INF, 0.0, 10.0], [-INF, -50.0, 50.0]]
RIGHT_LSE = [[1001.0, -1001.0, 0.0], [-INF, -INF, 11.0], [1.0, 50.0, -50.0]]


def _lse_close(got, ref):
    """LSE within 2e-6 plus two fp32 ulps of its magnitude (|lse| reaches 1001 here)."""
    got, ref = got.detach().cpu().double(), ref.double()
    both_inf = torch.isinf(ref) & (got == ref)
    diff = torch.where(both_inf, torch.zeros_like(ref), (got - ref).abs()).nan_to_num(float("inf"))
    bar = 2e-6 + 2.0 ** -22 * ref.abs().nan_to_num(0.0, posinf=0.0, neginf=0.0)
    return bool((diff <= bar).all())


def _rounding_bar(dtype, magnitude):
    """Half an ulp of `dtype` at `magnitude`, plus fp32 arithmetic slack."""
    if dtype == torch.float32:
        return 1e-6
    mantissa = 10 if dtype == torch.float16 else 7
    return 2.0 ** (torch.tensor(magnitude).log2().floor().item() - mantissa - 1) + 1e-6


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_pair_merge_of_strided_states_with_extreme_lse(device, dtype):
    """Strided state views, an LSE output that is a strided view, and a
    sentinel-filled output buffer (test_merge.py:10-27)."""
    g = torch.Generator().manual_seed(700)
    left = torch.randn(4, 3, 14, generator=g).to(dtype).to(device)[1:, :, 1::2]
    right = torch.randn(3, 6, 7, generator=g).to(dtype).to(device)[:, ::2]
    la, lb = torch.tensor(LEFT_LSE, device=device), torch.tensor(RIGHT_LSE, device=device)
    lse_store = torch.full((6, 6), 5.0, device=device)
    lse = lse_store[::2, 1::2]
    out_store = torch.full((3, 3, 14), 99.0, device=device, dtype=dtype)
    out = out_store[..., 1::2]
    merge_attn_states(out, left, la, right, lb, lse)
    ref, ref_lse = omerge.merge_pair(left, la, right, lb)
    assert max_err(out, ref) <= _rounding_bar(dtype, float(ref.abs().max()))
    assert _lse_close(lse, ref_lse)
    assert (out_store[..., ::2] == 99).all()
    assert (lse_store[1::2] == 5).all() and (lse_store[:, ::2] == 5).all()


def test_pair_merge_in_place_and_of_two_empty_states(device):
    """out and out_lse alias the left state; then two empty states with NaN
    payloads merge to 0 / -inf (test_merge.py:30-45)."""
    g = torch.Generator().manual_seed(710)
    left = torch.randn(2, 3, 4, generator=g).to(device)
    right = torch.randn(2, 3, 4, generator=g).to(device)
    la, lb = torch.zeros(3, 2, device=device), torch.ones(3, 2, device=device)
    ref, ref_lse = omerge.merge_pair(left, la, right, lb)
    merge_attn_states(left, left, la, right, lb, la)
    assert max_err(left, ref) <= 1e-6 and max_err(la, ref_lse) <= 1e-6
    left.fill_(float("nan"))
    right.fill_(float("nan"))
    la.fill_(-INF)
    lb.fill_(-INF)
    merge_attn_states(left, left, la, right, lb, la)
    assert torch.count_nonzero(left) == 0 and torch.isneginf(la).all()


def test_pair_merge_positive_infinity_takes_all_weight(device):
    """An LSE of +inf takes the whole weight (shared when both sides are +inf)."""
    g = torch.Generator().manual_seed(720)
    a = torch.randn(2, 2, 8, generator=g).to(device)
    b = torch.randn(2, 2, 8, generator=g).to(device)
    la = torch.tensor([[INF, 0.0], [INF, INF]], device=device)
    lb = torch.tensor([[0.0, INF], [INF, -INF]], device=device)
    out, lse = torch.empty_like(a), torch.empty_like(la)
    merge_attn_states(out, a, la, b, lb, lse)
    ref, ref_lse = omerge.merge_pair(a, la, b, lb)
    assert max_err(out, ref) <= 1e-6
    assert torch.equal(lse.cpu().double(), ref_lse)


@pytest.mark.parametrize("splits", [0, 1, 5, 70])
def test_merge_of_strided_partial_stacks(device, splits):
    """[S, T, H, D] partials as strided views; one (token, head) empty in every
    split and one split's payload NaN where its weight is 0
    (test_merge.py:48-62, plus a stack wider than one wavefront)."""
    g = torch.Generator().manual_seed(730 + splits)
    partial = torch.randn(splits, 4, 6, 14, generator=g).to(device)[:, 1:, ::2, 1::2]
    partial_lse = torch.randn(splits, 6, 6, generator=g).to(device)[:, ::2, 1::2]
    if splits:
        partial_lse[:, 0, 1] = -INF
        partial[:, 1, 0] = float("nan")
    out, lse = merge_partials(partial, partial_lse)
    ref, ref_lse = omerge.merge_partials(partial, partial_lse)
    assert max_err(out, ref) <= 2e-6 and max_err(lse, ref_lse) <= 2e-6
    if splits:
        assert torch.count_nonzero(out[1, 0]) == 0 and torch.isneginf(lse[0, 1])
