"""store_kvcache / append_kvcache / rotary on gfx950 vs the CPU oracle.

Ports flash_attn_mps tests/test_cache.py:10-140 (strides, skipped slots, bit
preservation, FP8 RNE/saturation table, append remapping, FP8 append, default
scale, rotary modes) and adds bit-exact checks of the vectorised paths at
benchmark-like shapes.  Cache bytes must match exactly.
"""
import numpy as np
import pytest
import torch

from flash_attn_mps_amd._cache import _unit_scale, append_kvcache, rotary, store_kvcache
from flash_attn_mps_amd import store_kvcache as public_store
from oracle import cache as ocache
from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu


def _bytes(t):
    return t.detach().cpu().contiguous().view(torch.uint8)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_store_strides_offsets_and_skipped_slots(device, dtype, index_dtype):
    k = torch.arange(5 * 4 * 12, device=device, dtype=torch.float32).to(dtype).reshape(5, 4, 12)[1:, ::2, 1::2]
    v = (k[..., :4] + 100).transpose(0, 1).contiguous().transpose(0, 1)
    kb = torch.full((4, 8, 4, 14), -3, device=device, dtype=dtype)
    vb = torch.full((4, 8, 4, 10), -5, device=device, dtype=dtype)
    kc, vc = kb[1:3, ::2, ::2, 1:13:2], vb[1:3, ::2, ::2, 1:9:2]
    ke, ve = kb.cpu(), vb.cpu()
    kev, vev = ke[1:3, ::2, ::2, 1:13:2], ve[1:3, ::2, ::2, 1:9:2]
    slots = torch.tensor([99, 6, 99, -1, 99, 0, 99, 3], dtype=index_dtype, device=device)[1::2]
    for t, slot in enumerate([6, -1, 0, 3]):
        if slot >= 0:
            kev[slot // 4, slot % 4] = k[t].cpu()
            vev[slot // 4, slot % 4] = v[t].cpu()
    store_kvcache(k, v, kc, vc, slots)
    assert torch.equal(kb.cpu(), ke)
    assert torch.equal(vb.cpu(), ve)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_store_preserves_float_bits(device, dtype):
    special = torch.tensor([0., -0., float("inf"), -float("inf"), float("nan"), 1e-30, -1e-30], dtype=dtype)
    k = special.reshape(1, 1, -1).to(device)
    cache = torch.empty((1, 1, 1, special.numel()), dtype=dtype, device=device)
    store_kvcache(k, k, cache, cache, torch.tensor([0], device=device))
    assert torch.equal(_bytes(cache).flatten(), special.view(torch.uint8))


def test_fp8_rne_saturation_and_scales(device):
    representable = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    ties = (representable[:-1] + representable[1:]) / 2
    values = torch.cat((representable, ties, -representable, -ties,
                        torch.tensor([1000., -1000., float("inf"), -float("inf")])))
    values = values[:, None, None].expand(-1, 2, 3).contiguous()
    scale = torch.tensor([.5, 2.])
    k = (values * scale[None, :, None]).to(device)
    v = (values * 4).to(device)
    kb = torch.empty((2, len(values), 2, 6), dtype=torch.float8_e4m3fn, device=device)
    vb = torch.empty_like(kb)
    kc, vc = kb[1:, :, :, ::2], vb[1:, :, :, ::2]
    store_kvcache(k, v, kc, vc, torch.arange(len(values), device=device), k_scale=scale.to(device), v_scale=4.)
    expected = values.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(kc.view(torch.uint8).cpu()[0], expected)
    assert torch.equal(vc.view(torch.uint8).cpu()[0], expected)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_fp8_store_random_matches_c_oracle(device, dtype):
    """Vectorised FP8 path (contiguous rows) and strided path vs the C codec."""
    g = torch.Generator().manual_seed(7)
    tokens, heads, dim, page = 777, 8, 256, 16
    x = (torch.randn(tokens, heads, dim, generator=g) * 40).to(dtype)
    x[3, 2, :8] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0., -0., 1e-9, 448., 464.])
    scale = torch.empty(heads).uniform_(0.01, 0.1, generator=g)
    pages = (tokens + page - 1) // page + 3
    perm = torch.randperm(pages * page, generator=g)[:tokens]
    perm[5] = -1
    for contiguous in (True, False):
        cache = torch.zeros(pages, page, heads, dim, dtype=torch.float8_e4m3fn, device=device)
        if contiguous:
            src = x.to(device)
        else:   # head-dim stride 2 and a head-major storage order
            buf = torch.zeros(heads, tokens, 2 * dim, dtype=dtype, device=device)
            buf[..., ::2] = x.to(device).transpose(0, 1)
            src = buf.transpose(0, 1)[..., ::2]
        store_kvcache(src, src, cache, cache, perm.to(device=device, dtype=torch.int64), k_scale=scale.to(device),
                      v_scale=scale.to(device))
        expected = ocache.store_kvcache(x, torch.zeros(pages, page, heads, dim, dtype=torch.float8_e4m3fn),
                                        perm, scale)
        assert torch.equal(_bytes(cache), _bytes(expected))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_bit_copy_large_random_permutation(device, dtype):
    """Benchmark-shaped scatter (16-token pages, permuted block table) is an exact copy."""
    g = torch.Generator().manual_seed(11)
    tokens, heads, dim, page = 4099, 8, 128, 16
    x = torch.randn(tokens, heads, dim, generator=g).to(dtype)
    pages = (tokens + page - 1) // page
    slots = torch.randperm(pages * page, generator=g)[:tokens].to(torch.int32)
    cache = torch.zeros(pages, page, heads, dim, dtype=dtype, device=device)
    public_store(x.to(device), x.to(device), cache, cache, slots.to(device))
    expected = ocache.store_kvcache(x, torch.zeros(pages, page, heads, dim, dtype=dtype), slots)
    assert torch.equal(_bytes(cache), _bytes(expected))


@pytest.mark.parametrize("paged", [False, True])
def test_append_batch_remapping_and_boundaries(device, paged):
    k = torch.arange(2 * 3 * 2 * 4, device=device, dtype=torch.float32).reshape(2, 3, 2, 4)
    v = k[..., :2] + 70
    kc = torch.full((6 if paged else 3, 4 if paged else 12, 2, 4), -1., device=device)
    vc = torch.full((*kc.shape[:-1], 2), -2., device=device)
    table = torch.tensor([[5, 0, 2], [1, 4, 3], [2, 3, 1]], device=device, dtype=torch.int32) if paged else None
    lengths = torch.tensor([3, 6], device=device, dtype=torch.int32)
    rows = torch.tensor([1, 0], device=device, dtype=torch.int32)
    ke = ocache.append_kvcache(k, kc, lengths, batch_index=rows, block_table=table)
    ve = ocache.append_kvcache(v, vc, lengths, batch_index=rows, block_table=table)
    append_kvcache(k, v, kc, vc, lengths, cache_batch_idx=rows,
                   cache_leftpad=torch.tensor([2, 1], device=device), block_table=table)
    assert torch.equal(kc.cpu(), ke)
    assert torch.equal(vc.cpu(), ve)
    assert torch.equal(lengths.cpu(), torch.tensor([3, 6], dtype=torch.int32))


def test_append_fp8_scales(device):
    k = torch.randn((2, 2, 3, 5), device=device)
    v = torch.randn((2, 2, 3, 7), device=device)
    kc = torch.zeros((2, 4, 3, 5), dtype=torch.float8_e4m3fn, device=device)
    vc = torch.zeros((2, 4, 3, 7), dtype=torch.float8_e4m3fn, device=device)
    scale = torch.tensor([.5, 1., 2.], device=device)
    append_kvcache(k, v, kc, vc, 1, k_scale=scale, v_scale=2.)
    ke = (k.cpu() / scale.cpu()[None, None, :, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    ve = (v.cpu() / 2).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(kc.cpu()[:, 1:3].contiguous().view(torch.uint8), ke)
    assert torch.equal(vc.cpu()[:, 1:3].contiguous().view(torch.uint8), ve)


def test_fp8_default_scale_with_float16_default_dtype(device):
    old_dtype = torch.get_default_dtype()
    _unit_scale.cache_clear()
    try:
        torch.set_default_dtype(torch.float16)
        k = torch.tensor([[[1., 2., 3., 4.]]], device=device)
        cache = torch.empty((1, 1, 1, 4), device=device, dtype=torch.float8_e4m3fn)
        store_kvcache(k, k, cache, cache, torch.tensor([0], device=device))
        expected = k.cpu().to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(cache.view(torch.uint8).cpu()[0], expected)
    finally:
        torch.set_default_dtype(old_dtype)
        _unit_scale.cache_clear()


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("mode", ["global", "causal", "local"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_rotary_modes_strides_and_partial_head(device, interleaved, mode, dtype):
    q = torch.randn((2, 3, 4, 16), device=device).to(dtype)[..., 1::2]
    k = torch.randn((2, 2, 2, 16), device=device).to(dtype)[..., 1::2]
    angles = torch.randn((20, 4), device=device)[:, ::2]
    cos, sin = angles.cos(), angles.sin()
    lengths = torch.tensor([2, 7], device=device)
    window = (3, -1) if mode == "local" else [-1, -1]
    qr, kr = rotary(q, k, cos, sin, lengths, rotary_interleaved=interleaved, causal=mode == "causal",
                    window_size=window)
    qe = ocache.rotary(q, cos, sin, lengths, interleaved, mode != "global").to(dtype)
    ke = ocache.rotary(k, cos, sin, lengths, interleaved, True).to(dtype)
    tol = dict(rtol=1e-5, atol=5e-7) if dtype == torch.float32 else dict(rtol=8e-3, atol=8e-3)
    torch.testing.assert_close(qr.cpu(), qe, **tol)
    torch.testing.assert_close(kr.cpu(), ke, **tol)
    assert torch.equal(qr.cpu()[..., 4:], q.cpu()[..., 4:])


def test_fp8_hardware_decode_matches_codec(device):
    """Every E4M3 code decoded by the attention kernels equals the C codec:
    a one-hot value row per code reads back the decoded value exactly."""
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes != 127) & (codes != 255)]
    expect = torch.from_numpy(ofp8.decode(codes.numpy()))
    # K = 0 makes all weights equal; V carries the code under test in dim 0 of
    # a single key, so the output is exactly decode(code) * 1.0.
    from flash_attn_mps_amd._decode import decode_attention
    n = codes.numel()
    q = torch.zeros(n, 1, 64, device=device, dtype=torch.float32)
    kraw = torch.zeros(n, 16, 1, 64, dtype=torch.uint8)
    vraw = torch.zeros(n, 16, 1, 64, dtype=torch.uint8)
    vraw[:, 0, 0, :] = codes[:, None]
    k = kraw.view(torch.float8_e4m3fn).to(device)
    v = vraw.view(torch.float8_e4m3fn).to(device)
    cq = torch.arange(n + 1, device=device, dtype=torch.int32)
    used = torch.ones(n, device=device, dtype=torch.int32)
    table = torch.arange(n, device=device, dtype=torch.int32).reshape(n, 1)
    out = torch.empty(n, 1, 64, device=device, dtype=torch.float32)
    decode_attention(q, k, v, cu_seqlens_q=cq, seqused_k=used, max_seqlen_k=1, block_table=table, out=out)
    assert torch.equal(out.cpu()[:, 0, 0], expect)
    assert torch.equal(out.cpu()[:, 0, 1], expect)
