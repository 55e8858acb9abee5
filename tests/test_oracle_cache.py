"""The CPU cache oracle (oracle/cache.py) against index_copy_ scatter, torch's
float8 cast, literal known positions and complex-number rotation (CPU only)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import cache as ocache
from oracle.attention import attention

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_store_equals_index_copy(dtype):
    """cache.view(N * P, H, D).index_copy_(0, valid slots, x): slot < 0 and
    slot >= N * P are skipped."""
    g = torch.Generator().manual_seed(1)
    pages, page, h, d = 6, 4, 2, 5
    x = torch.randn(10, h, d, generator=g).to(dtype)
    slots = torch.randperm(pages * page, generator=g)[:10]
    slots[3], slots[7] = -1, pages * page + 2
    cache = torch.randn(pages, page, h, d, generator=g).to(dtype)
    got = ocache.store_kvcache(x, cache, slots)
    valid = (slots >= 0) & (slots < pages * page)
    want = cache.clone().view(pages * page, h, d).index_copy_(0, slots[valid], x[valid]).view_as(cache)
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_store_preserves_special_bits(dtype):
    """flash_attn_mps tests/test_cache.py:30-36 (plus a NaN payload)."""
    special = torch.tensor([0., -0., float("inf"), -float("inf"), float("nan"), 1e-30, -1e-30], dtype=dtype)
    bits = special.view(torch.int16 if dtype != torch.float32 else torch.int32).clone()
    bits[4] = bits[4] | 1                                            # NaN with a payload bit
    special = bits.view(dtype)
    cache = torch.zeros(1, 1, 1, special.numel(), dtype=dtype)
    got = ocache.store_kvcache(special.reshape(1, 1, -1), cache, torch.tensor([0]))
    assert torch.equal(got.view(torch.uint8).flatten(), special.view(torch.uint8))


def test_store_fp8_equals_torch_cast_of_scaled_values():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(12, 3, 8, generator=g).to(torch.bfloat16) * 30
    scale = torch.tensor([0.5, 0.05, 2.0])
    cache = torch.zeros(4, 4, 3, 8, dtype=torch.float8_e4m3fn)
    slots = torch.arange(12) + 2
    got = ocache.store_kvcache(x, cache, slots, scale=scale)
    codes = (x.float() / scale[None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    want = cache.view(torch.uint8).clone().view(16, 3, 8).index_copy_(0, slots, codes).view(4, 4, 3, 8)
    assert torch.equal(got.view(torch.uint8), want)


@pytest.mark.parametrize("paged", [False, True])
def test_append_known_positions(paged):
    """flash_attn_mps tests/test_cache.py:57-75 with the landing positions
    written out: lengths [3, 6], three new tokens, batch rows [1, 0] or the
    page table [[5, 0, 2], [1, 4, 3]] with 4-token pages."""
    k = torch.arange(2 * 3 * 2 * 4, dtype=torch.float32).reshape(2, 3, 2, 4)
    cache = torch.full((6 if paged else 3, 4 if paged else 12, 2, 4), -1.0)
    table = torch.tensor([[5, 0, 2], [1, 4, 3], [2, 3, 1]], dtype=torch.int32) if paged else None
    got = ocache.append_kvcache(k, cache, torch.tensor([3, 6]), batch_index=torch.tensor([1, 0]),
                                block_table=table)
    if paged:
        landing = {(0, 0): (5, 3), (0, 1): (0, 0), (0, 2): (0, 1), (1, 0): (4, 2), (1, 1): (4, 3), (1, 2): (3, 0)}
    else:
        landing = {(0, 0): (1, 3), (0, 1): (1, 4), (0, 2): (1, 5), (1, 0): (0, 6), (1, 1): (0, 7), (1, 2): (0, 8)}
    want = cache.clone()
    for (b, j), (blk, off) in landing.items():
        want[blk, off] = k[b, j]
    assert torch.equal(got, want)


def test_append_out_of_range_is_skipped():
    k = torch.ones(1, 3, 1, 2)
    cache = torch.zeros(1, 4, 1, 2)
    got = ocache.append_kvcache(k, cache, torch.tensor([2]))          # positions 2, 3, 4: 4 is past the end
    assert got[0, :, 0, 0].tolist() == [0.0, 0.0, 1.0, 1.0]


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("advance", [True, False])
def test_rotary_equals_complex_rotation(interleaved, advance):
    """Interleaved pairs rotate as complex numbers x * e^{i theta}; split halves
    follow out = x cos + rotate_half(x) sin.  Dims past the rotary width are
    untouched."""
    g = torch.Generator().manual_seed(3)
    b, s, h, d, half = 2, 3, 2, 10, 3
    x = torch.randn(b, s, h, d, generator=g, dtype=torch.float64)
    theta = torch.randn(12, half, generator=g, dtype=torch.float64)
    lengths = torch.tensor([1, 5])
    got = ocache.rotary(x, theta.cos(), theta.sin(), lengths, interleaved, advance)
    want = x.clone()
    for bi in range(b):
        for j in range(s):
            ang = theta[int(lengths[bi]) + (j if advance else 0)]
            if interleaved:
                z = torch.view_as_complex(x[bi, j, :, :2 * half].reshape(h, half, 2).contiguous())
                want[bi, j, :, :2 * half] = torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(h, -1)
            else:
                xr = x[bi, j, :, :2 * half]
                cos, sin = torch.cat((ang.cos(), ang.cos())), torch.cat((ang.sin(), ang.sin()))
                rot = torch.cat((-xr[:, half:], xr[:, :half]), dim=-1)
                want[bi, j, :, :2 * half] = xr * cos + rot * sin
    torch.testing.assert_close(got, want, atol=1e-14, rtol=0)
    assert torch.equal(got[..., 2 * half:], x[..., 2 * half:])


def test_attention_matches_sdpa_golden():
    """tests/golden/sdpa.npz: a varlen GQA causal case whose outputs torch SDPA wrote."""
    g = np.load(GOLDEN / "sdpa.npz")
    q, k, v = (torch.from_numpy(g[n]) for n in ("q", "k", "v"))
    cuq = torch.tensor(np.concatenate(([0], np.cumsum(g["q_lens"]))), dtype=torch.int32)
    cuk = torch.tensor(np.concatenate(([0], np.cumsum(g["k_lens"]))), dtype=torch.int32)
    out, _ = attention(q, k, v, cuq, cuk, causal=True, scale=float(g["scale"]))
    torch.testing.assert_close(out, torch.from_numpy(g["out"]), atol=1e-12, rtol=0)
