"""The CPU merge oracle (oracle/merge.py) against log-add-exp closed forms and
the reference's merge tables (flash_attn_mps tests/test_merge.py); CPU only."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.merge import merge_pair, merge_partials

GOLDEN = Path(__file__).resolve().parent / "golden" / "merge.npz"


def test_pair_merge_extreme_lse_table():
    """test_merge.py:14-27: LSEs of +-1000, +-50, -inf on either side."""
    g = np.load(GOLDEN)
    out, lse = merge_pair(torch.from_numpy(g["left"]), torch.from_numpy(g["left_lse"]),
                          torch.from_numpy(g["right"]), torch.from_numpy(g["right_lse"]))
    torch.testing.assert_close(lse, torch.from_numpy(g["lse"]), atol=1e-12, rtol=0)
    torch.testing.assert_close(out, torch.from_numpy(g["out"]), atol=1e-12, rtol=0)


def test_pair_merge_closed_form_and_empty_nan_payload():
    """test_merge.py:30-45: lse 0 and 1 weight 1 : e; both -inf -> 0 and -inf
    even when the payloads are NaN."""
    left = torch.randn(2, 3, 4, dtype=torch.float64)
    right = torch.randn_like(left)
    la, lb = torch.zeros(3, 2, dtype=torch.float64), torch.ones(3, 2, dtype=torch.float64)
    out, lse = merge_pair(left, la, right, lb)
    torch.testing.assert_close(out, (left + right * np.e) / (1 + np.e), atol=1e-14, rtol=0)
    torch.testing.assert_close(lse, torch.full((3, 2), np.log1p(np.e), dtype=torch.float64))
    nan = torch.full_like(left, float("nan"))
    ninf = torch.full_like(la, -float("inf"))
    out, lse = merge_pair(nan, ninf, nan, ninf)
    assert torch.equal(out, torch.zeros_like(out)) and bool(torch.isneginf(lse).all())


@pytest.mark.parametrize("splits", [0, 1, 5])
def test_merge_partials_noncontiguous_empty_and_nan(splits):
    """test_merge.py:48-61: logsumexp LSE, weights exp(l - lse); a -inf split
    with a NaN payload is ignored."""
    g = torch.Generator().manual_seed(splits)
    p = torch.randn((splits, 4, 6, 14), generator=g, dtype=torch.float64)[:, 1:, ::2, 1::2]
    l = torch.randn((splits, 6, 6), generator=g, dtype=torch.float64)[:, ::2, 1::2]
    if splits:
        l[:, 0, 1] = -float("inf")
        p[:, 1, 0] = float("nan")
    out, lse = merge_partials(p, l)
    expected_lse = torch.logsumexp(l, dim=0)
    weights = (l - expected_lse).exp().nan_to_num(0).transpose(1, 2).unsqueeze(-1)
    expected = (weights * torch.where(weights > 0, p, torch.zeros_like(p))).sum(0)
    torch.testing.assert_close(out, expected, atol=1e-13, rtol=0)
    torch.testing.assert_close(lse, expected_lse, atol=1e-13, rtol=0)


def test_plus_inf_lse_takes_exclusive_weight():
    """A +inf LSE is the limit of a dominating split: the +inf splits share the
    weight equally, as with a huge finite LSE; others get none."""
    o = torch.randn(3, 2, 1, 5, dtype=torch.float64)
    lse = torch.tensor([[[float("inf"), 0.0]], [[3.0, 1.0]], [[float("inf"), 2.0]]],
                       dtype=torch.float64)                    # [S=3, H=1, T=2]
    out, merged = merge_partials(o, lse)
    assert out.shape == (2, 1, 5) and merged.shape == (1, 2)
    big = torch.where(torch.isinf(lse), torch.full_like(lse, 700.0), lse)
    out_big, _ = merge_partials(o, big)
    torch.testing.assert_close(out, out_big, atol=1e-12, rtol=0)
    torch.testing.assert_close(out[0, 0], (o[0, 0, 0] + o[2, 0, 0]) / 2)
    assert merged[0, 0] == float("inf")
