"""The CPU attention oracle against facts independent of its formula (CPU only).

The checks live in oracle_pins.py: torch SDPA on every feature it can
express, closed forms, feature identities and the reference's empty-KV
golden values.  test_oracle_mutants.py shows each check has teeth.
"""
import pytest
import torch

import oracle_pins
from oracle.attention import attention, flops


@pytest.mark.parametrize("check", oracle_pins.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_attention_pinned(check):
    check(attention)


def test_flops_counts_visible_pairs():
    """flops() = brute-force count of visible (query, key) pairs x Hq x 2(Dqk + Dv)."""
    for q_lens, k_lens, window in (([5, 1, 8], [5, 9, 3], -1), ([4, 6], [10, 6], 2)):
        pairs = 0
        for n, m in zip(q_lens, k_lens):
            for i in range(n):
                for j in range(m):
                    d = (m - n + i) - j
                    pairs += d >= 0 and (window < 0 or d <= window)
        assert flops(q_lens, k_lens, 3, 16, 8, window_left=window) == pairs * 3 * 2 * 24
    # equal lengths, full causal: L (L + 1) / 2 pairs per request
    assert flops([7, 100], [7, 100], 1, 1, 1) == (7 * 8 // 2 + 100 * 101 // 2) * 2 * 2


def test_float32_mode_matches_float64():
    """dtype=float32 (the CPU baseline's precision) stays within fp32 rounding of float64."""
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(64, 4, 32, generator=g) for _ in range(3))
    cu = torch.tensor([0, 40, 64], dtype=torch.int32)
    o64, l64 = attention(q, k, v, cu, cu, causal=True)
    o32, l32 = attention(q, k, v, cu, cu, causal=True, dtype=torch.float32)
    assert o32.dtype == torch.float32
    torch.testing.assert_close(o32.double(), o64, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(l32.double(), l64, atol=1e-5, rtol=1e-5)
