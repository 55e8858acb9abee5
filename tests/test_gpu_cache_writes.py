"""KV-cache writes and rotary embedding on gfx950 against the CPU oracle
(oracle/cache.py, and the C E4M3 codec in oracle/fp8_e4m3.c).

Strides, skipped slots, special float bits, the FP8 rounding/saturation
table, append remapping and rotary modes are data from flash_attn_mps
tests/test_cache.py (cited per case).  Every cache byte must match exactly;
rotary outputs are within one rounding of the fp64 rotation.
"""
import pytest
import torch

import flash_attn_mps_amd as fa
from flash_attn_mps_amd._cache import append_kvcache, rotary, store_kvcache
from harness import decode_attention, max_err
from oracle import cache as ocache
from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu

INF = float("inf")


def _bytes(t):
    return t.detach().cpu().contiguous().view(torch.uint8)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_store_through_views_skipping_negative_slots(device, dtype, slot_dtype):
    """Strided K/V and cache views with storage offsets, a strided slot
    vector with a -1 entry (test_cache.py:10-27: slots 6, -1, 0, 3)."""
    k = torch.arange(5 * 4 * 12, dtype=torch.float32).to(dtype).reshape(5, 4, 12).to(device)[1:, ::2, 1::2]
    v = (k[..., :4] + 100).transpose(0, 1).contiguous().transpose(0, 1)
    k_store = torch.full((4, 8, 4, 14), -3.0, device=device, dtype=dtype)
    v_store = torch.full((4, 8, 4, 10), -5.0, device=device, dtype=dtype)
    k_cache, v_cache = k_store[1:3, ::2, ::2, 1:13:2], v_store[1:3, ::2, ::2, 1:9:2]
    slots = torch.tensor([99, 6, 99, -1, 99, 0, 99, 3], dtype=slot_dtype, device=device)[1::2]
    expect_k, expect_v = k_store.cpu(), v_store.cpu()
    ek, ev = expect_k[1:3, ::2, ::2, 1:13:2], expect_v[1:3, ::2, ::2, 1:9:2]
    for t, slot in enumerate((6, -1, 0, 3)):
        if slot >= 0:
            ek[slot // 4, slot % 4], ev[slot // 4, slot % 4] = k[t].cpu(), v[t].cpu()
    store_kvcache(k, v, k_cache, v_cache, slots)
    assert torch.equal(_bytes(k_store), _bytes(expect_k)) and torch.equal(_bytes(v_store), _bytes(expect_v))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_same_dtype_store_keeps_every_bit(device, dtype):
    """Signed zeros, infinities, NaN and tiny values are copied bit for bit
    (test_cache.py:30-36)."""
    special = torch.tensor([0.0, -0.0, INF, -INF, float("nan"), 1e-30, -1e-30], dtype=dtype)
    x = special.reshape(1, 1, -1).to(device)
    cache = torch.empty(1, 1, 1, special.numel(), dtype=dtype, device=device)
    store_kvcache(x, x, cache, cache, torch.tensor([0], device=device))
    assert torch.equal(_bytes(cache).flatten(), special.view(torch.uint8))


def test_fp8_store_rounding_saturation_and_scales(device):
    """Every positive code, every midpoint between neighbours (ties to even),
    their negatives, +-1000 and +-inf (saturate to +-448), with per-head K
    scales 0.5 / 2 and a scalar V scale 4; caches are strided views
    (test_cache.py:39-54)."""
    codes = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (codes[:-1] + codes[1:]) / 2
    values = torch.cat((codes, mids, -codes, -mids, torch.tensor([1000.0, -1000.0, INF, -INF])))
    values = values[:, None, None].expand(-1, 2, 3).contiguous()
    k_scale = torch.tensor([0.5, 2.0])
    k = (values * k_scale[None, :, None]).to(device)
    v = (values * 4).to(device)
    k_store = torch.empty(2, len(values), 2, 6, dtype=torch.float8_e4m3fn, device=device)
    v_store = torch.empty_like(k_store)
    k_cache, v_cache = k_store[1:, :, :, ::2], v_store[1:, :, :, ::2]
    store_kvcache(k, v, k_cache, v_cache, torch.arange(len(values), device=device), k_scale=k_scale.to(device),
                  v_scale=4.0)
    expected = torch.from_numpy(ofp8.encode(values.numpy()))
    assert torch.equal(_bytes(k_cache)[0], expected) and torch.equal(_bytes(v_cache)[0], expected)
    # The C codec agrees with torch's own cast on this table (saturating first).
    assert torch.equal(expected, values.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp8_row_store_codes_midpoints_and_every_bf16_pattern(device, dtype):
    """The row kernel (contiguous [T, 8, 256] rows), whose E4M3 bytes come
    from the hardware conversion: every code and every midpoint between
    neighbours (ties to even) with their negatives, +-1000, +-inf and NaN,
    under power-of-two per-head scales (exact quotients), then all 65536
    bf16 bit patterns under scales 1, 2^-4 and 0.0173; bytes against the C
    codec."""
    heads, dim, page = 8, 256, 16
    codes = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (codes[:-1] + codes[1:]) / 2
    table = torch.cat((codes, mids, -codes, -mids, torch.tensor([1000.0, -1000.0, INF, -INF, float("nan")])))
    row = table.repeat(-(-heads * dim // len(table)))[: heads * dim].reshape(heads, dim)
    scale = torch.tensor([0.5, 2.0, 1.0, 0.25, 4.0, 0.125, 8.0, 1.0])
    rows = [row * scale[:, None]]
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    x = torch.cat((torch.stack(rows), bits.reshape(-1, heads, dim))).to(dtype)
    tokens = x.shape[0]
    for s in (scale, torch.full((heads,), 2.0 ** -4), torch.full((heads,), 0.0173)):
        pages = -(-tokens // page)
        slots = torch.arange(tokens)
        cache = torch.zeros(pages, page, heads, dim, dtype=torch.float8_e4m3fn, device=device)
        store_kvcache(x.to(device), x.to(device), cache, cache, slots.to(device), k_scale=s.to(device),
                      v_scale=s.to(device))
        expected = ocache.store_kvcache(x, torch.zeros(pages, page, heads, dim, dtype=torch.float8_e4m3fn), slots, s)
        assert torch.equal(_bytes(cache), _bytes(expected)), f"scale {s.tolist()}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("contiguous", [True, False])
def test_fp8_store_of_random_rows_matches_the_c_codec(device, dtype, contiguous):
    """777 tokens x 8 heads x 256 dims at 40x scale with specials, per-head
    scales U[0.01, 0.1], a skipped slot; contiguous rows (vector path) and a
    head-major stride-2 view (element path)."""
    g = torch.Generator().manual_seed(740)
    tokens, heads, dim, page = 777, 8, 256, 16
    x = (torch.randn(tokens, heads, dim, generator=g) * 40).to(dtype)
    x[3, 2, :8] = torch.tensor([float("nan"), INF, -INF, 0.0, -0.0, 1e-9, 448.0, 464.0])
    scale = torch.empty(heads).uniform_(0.01, 0.1, generator=g)
    pages = -(-tokens // page) + 3
    slots = torch.randperm(pages * page, generator=g)[:tokens]
    slots[5] = -1
    cache = torch.zeros(pages, page, heads, dim, dtype=torch.float8_e4m3fn, device=device)
    if contiguous:
        src = x.to(device)
    else:
        store = torch.zeros(heads, tokens, 2 * dim, dtype=dtype, device=device)
        store[..., ::2] = x.to(device).transpose(0, 1)
        src = store.transpose(0, 1)[..., ::2]
    store_kvcache(src, src, cache, cache, slots.to(device), k_scale=scale.to(device), v_scale=scale.to(device))
    expected = ocache.store_kvcache(x, torch.zeros(pages, page, heads, dim, dtype=torch.float8_e4m3fn), slots, scale)
    assert torch.equal(_bytes(cache), _bytes(expected))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_scatter_over_a_permuted_pool(device, dtype):
    """Benchmark-shaped scatter (16-token pages, random slot permutation)
    through the public entry point is an exact copy."""
    g = torch.Generator().manual_seed(750)
    tokens, heads, dim, page = 4099, 8, 128, 16
    x = torch.randn(tokens, heads, dim, generator=g).to(dtype)
    pages = -(-tokens // page)
    slots = torch.randperm(pages * page, generator=g)[:tokens].to(torch.int32)
    cache = torch.zeros(pages, page, heads, dim, dtype=dtype, device=device)
    fa.store_kvcache(x.to(device), x.to(device), cache, cache, slots.to(device))
    expected = ocache.store_kvcache(x, torch.zeros(pages, page, heads, dim, dtype=dtype), slots)
    assert torch.equal(_bytes(cache), _bytes(expected))


@pytest.mark.parametrize("paged", [False, True])
def test_append_with_row_remap_and_page_tables(device, paged):
    """Three new tokens per request at lengths 3 and 6, rows remapped [1, 0]
    (dense) or through a 3x3 page table of 4-token pages; leftpad does not
    move the writes and lengths stay unchanged (test_cache.py:57-75)."""
    k = torch.arange(2 * 3 * 2 * 4, dtype=torch.float32).reshape(2, 3, 2, 4).to(device)
    v = k[..., :2] + 70
    k_cache = torch.full((6 if paged else 3, 4 if paged else 12, 2, 4), -1.0, device=device)
    v_cache = torch.full((*k_cache.shape[:-1], 2), -2.0, device=device)
    table = torch.tensor([[5, 0, 2], [1, 4, 3], [2, 3, 1]], device=device, dtype=torch.int32) if paged else None
    lengths = torch.tensor([3, 6], device=device, dtype=torch.int32)
    rows = torch.tensor([1, 0], device=device, dtype=torch.int32)
    expect_k = ocache.append_kvcache(k, k_cache, lengths, None if paged else rows, table)
    expect_v = ocache.append_kvcache(v, v_cache, lengths, None if paged else rows, table)
    append_kvcache(k, v, k_cache, v_cache, lengths, cache_batch_idx=rows,
                   cache_leftpad=torch.tensor([2, 1], device=device), block_table=table)
    assert torch.equal(k_cache.cpu(), expect_k) and torch.equal(v_cache.cpu(), expect_v)
    assert lengths.tolist() == [3, 6]


def test_append_into_fp8_caches(device):
    """Per-head K scales and a scalar V scale, appended at position 1 of every
    row (test_cache.py:78-88)."""
    g = torch.Generator().manual_seed(760)
    k = torch.randn(2, 2, 3, 5, generator=g).to(device)
    v = torch.randn(2, 2, 3, 7, generator=g).to(device)
    k_cache = torch.zeros(2, 4, 3, 5, dtype=torch.float8_e4m3fn, device=device)
    v_cache = torch.zeros(2, 4, 3, 7, dtype=torch.float8_e4m3fn, device=device)
    k_scale = torch.tensor([0.5, 1.0, 2.0], device=device)
    append_kvcache(k, v, k_cache, v_cache, 1, k_scale=k_scale, v_scale=2.0)
    expect_k = ocache.append_kvcache(k, torch.zeros(2, 4, 3, 5, dtype=torch.float8_e4m3fn), 1, scale=k_scale)
    expect_v = ocache.append_kvcache(v, torch.zeros(2, 4, 3, 7, dtype=torch.float8_e4m3fn), 1, scale=2.0)
    assert torch.equal(_bytes(k_cache), _bytes(expect_k)) and torch.equal(_bytes(v_cache), _bytes(expect_v))


def test_fp8_store_default_scale_under_a_half_default_dtype(device):
    """No scale means 1.0 in fp32 even when torch's default dtype is fp16
    (test_cache.py:91-103)."""
    previous = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.float16)
        x = torch.tensor([[[1.0, 2.0, 3.0, 4.0]]], device=device)
        cache = torch.empty(1, 1, 1, 4, device=device, dtype=torch.float8_e4m3fn)
        store_kvcache(x, x, cache, cache, torch.tensor([0], device=device))
        assert torch.equal(_bytes(cache)[0], x.cpu().float().to(torch.float8_e4m3fn).view(torch.uint8))
    finally:
        torch.set_default_dtype(previous)


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("mode", ["global", "causal", "local"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_rotary_modes_on_strided_heads(device, interleaved, mode, dtype):
    """Rotary dim 4 of 8 (stride-2 views), queries fixed at the old length for
    global attention and advancing for causal/local (test_cache.py:129-140)."""
    g = torch.Generator().manual_seed(770)
    q = torch.randn(2, 3, 4, 16, generator=g).to(dtype).to(device)[..., 1::2]
    k = torch.randn(2, 2, 2, 16, generator=g).to(dtype).to(device)[..., 1::2]
    angles = torch.randn(20, 4, generator=g).to(device)[:, ::2]
    cos, sin = angles.cos(), angles.sin()
    lengths = torch.tensor([2, 7], device=device)
    window = (3, -1) if mode == "local" else (-1, -1)
    q_rot, k_rot = rotary(q, k, cos, sin, lengths, rotary_interleaved=interleaved, causal=mode == "causal",
                          window_size=window)
    q_ref = ocache.rotary(q, cos, sin, lengths, interleaved, mode != "global")
    k_ref = ocache.rotary(k, cos, sin, lengths, interleaved, True)
    for got, ref in ((q_rot, q_ref), (k_rot, k_ref)):
        bar = 1e-6 if dtype == torch.float32 else 2.0 ** -(11 if dtype == torch.float16 else 8) * 4
        assert max_err(got, ref) <= bar
    assert torch.equal(q_rot[..., 4:], q[..., 4:])


def test_decode_kernel_widens_every_fp8_code_exactly(device):
    """Each finite E4M3 code, as the value of a single key, comes back from
    the decode kernel exactly as the C codec decodes it."""
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes != 0x7F) & (codes != 0xFF)]
    n = codes.numel()
    k_raw = torch.zeros(n, 16, 1, 64, dtype=torch.uint8)
    v_raw = torch.zeros(n, 16, 1, 64, dtype=torch.uint8)
    v_raw[:, 0, 0, :] = codes[:, None]
    k, v = (t.view(torch.float8_e4m3fn).to(device) for t in (k_raw, v_raw))
    q = torch.zeros(n, 1, 64, device=device, dtype=torch.bfloat16)
    out = torch.empty(n, 1, 64, device=device, dtype=torch.float32)
    decode_attention(q, k, v, cu_seqlens_q=torch.arange(n + 1, device=device, dtype=torch.int32),
                     seqused_k=torch.ones(n, device=device, dtype=torch.int32), max_seqlen_k=1,
                     block_table=torch.arange(n, device=device, dtype=torch.int32).reshape(n, 1), out=out)
    expected = torch.from_numpy(ofp8.decode(codes.numpy()))
    assert torch.equal(out.cpu()[:, 0, 0], expected) and torch.equal(out.cpu()[:, 0, 63], expected)
