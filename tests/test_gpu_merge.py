"""merge_attn_states / _merge_partials on gfx950 vs closed forms.

Ports flash_attn_mps tests/test_merge.py:10-61: strided pair merge with
extreme LSEs (+-1000, -inf, +inf-free table), in-place aliasing, NaN payloads
of empty states, N-way merge of non-contiguous partials including zero splits.
"""
import pytest
import torch

from flash_attn_mps_amd._merge import _merge_partials, merge_attn_states
from oracle import merge as omerge

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_pair_merge_strided_and_extreme_lse(device, dtype):
    left = torch.randn((4, 3, 14), device=device).to(dtype)[1:, :, 1::2]
    right = torch.randn((3, 6, 7), device=device).to(dtype)[:, ::2]
    la = torch.tensor([[1000., -1000., -float("inf")], [-float("inf"), 0., 10.], [-float("inf"), -50., 50.]], device=device)
    lb = torch.tensor([[1001., -1001., 0.], [-float("inf"), -float("inf"), 11.], [1., 50., -50.]], device=device)
    lse_base = torch.empty((6, 6), device=device)
    lse = lse_base[::2, 1::2]
    out_base = torch.full((3, 3, 14), 99., device=device, dtype=dtype)
    out = out_base[..., 1::2]
    merge_attn_states(out, left, la, right, lb, lse)
    le = torch.logaddexp(la.cpu().double(), lb.cpu().double())
    wa = (la.cpu().double() - le).exp().nan_to_num(0).T.unsqueeze(-1)
    wb = (lb.cpu().double() - le).exp().nan_to_num(0).T.unsqueeze(-1)
    expected = (wa * left.cpu().double() + wb * right.cpu().double()).to(dtype)
    tol = dict(rtol=8e-3, atol=8e-3) if dtype == torch.bfloat16 else dict(rtol=2e-3, atol=2e-6)
    torch.testing.assert_close(out.cpu(), expected, **tol)
    torch.testing.assert_close(lse.cpu(), le.float(), rtol=1e-6, atol=2e-6)
    assert torch.equal(out_base.cpu()[..., ::2], torch.full((3, 3, 7), 99., dtype=dtype))
    o_out, o_lse = omerge.merge_pair(left, la, right, lb)
    torch.testing.assert_close(out.cpu().double(), o_out, **tol)


def test_merge_inplace_and_empty_nan_payload(device):
    left = torch.randn((2, 3, 4), device=device)
    right = torch.randn_like(left)
    la = torch.zeros((3, 2), device=device)
    lb = torch.ones_like(la)
    expected = (left.cpu() + right.cpu() * torch.e) / (1 + torch.e)
    merge_attn_states(left, left, la, right, lb, la)
    torch.testing.assert_close(left.cpu(), expected)
    torch.testing.assert_close(la.cpu(), torch.full((3, 2), torch.log(torch.tensor(1 + torch.e))))
    left.fill_(float("nan"))
    right.fill_(float("nan"))
    la.fill_(-float("inf"))
    lb.fill_(-float("inf"))
    merge_attn_states(left, left, la, right, lb, la)
    assert torch.equal(left.cpu(), torch.zeros_like(left.cpu()))
    assert torch.isneginf(la.cpu()).all()


def test_merge_positive_infinity_takes_all_weight(device):
    a = torch.randn((2, 2, 8), device=device)
    b = torch.randn_like(a)
    la = torch.tensor([[float("inf"), 0.], [float("inf"), float("inf")]], device=device)
    lb = torch.tensor([[0., float("inf")], [float("inf"), -float("inf")]], device=device)
    out = torch.empty_like(a)
    lse = torch.empty_like(la)
    merge_attn_states(out, a, la, b, lb, lse)
    o_out, o_lse = omerge.merge_pair(a, la, b, lb)
    torch.testing.assert_close(out.cpu().double(), o_out, rtol=1e-6, atol=1e-6)
    assert torch.equal(lse.cpu().double(), o_lse)


@pytest.mark.parametrize("splits", [0, 1, 5])
def test_merge_partials_noncontiguous_and_empty(device, splits):
    p = torch.randn((splits, 4, 6, 14), device=device)[:, 1:, ::2, 1::2]
    l = torch.randn((splits, 6, 6), device=device)[:, ::2, 1::2]
    if splits:
        l[:, 0, 1] = -float("inf")
        p[:, 1, 0] = float("nan")
    out, lse = _merge_partials(p, l)
    expected_lse = torch.logsumexp(l.cpu().double(), dim=0)
    weights = (l.cpu().double() - expected_lse).exp().nan_to_num(0).transpose(1, 2).unsqueeze(-1)
    values = torch.where(weights > 0, p.cpu().double(), 0.)
    expected = (weights * values).sum(0).float()
    torch.testing.assert_close(out.cpu(), expected, rtol=1e-5, atol=5e-7)
    torch.testing.assert_close(lse.cpu(), expected_lse.float(), rtol=1e-5, atol=5e-7)
    o_out, o_lse = omerge.merge_partials(p, l)
    torch.testing.assert_close(out.cpu().double(), o_out, rtol=1e-5, atol=5e-7)
