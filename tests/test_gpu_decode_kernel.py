"""Single-query split-KV decode on gfx950 against the CPU oracle.

Part of the cases are data from flash_attn_mps tests/test_decode.py (cited
per case); the rest exercise this build's decode kernel: its 16-token page
walk, padded head dims, head-group tiles and ALiBi.  Checks: parity bar
(fp16 2e-3, bf16 1e-2, fp32 1e-4, LSE 1e-4 max-abs), NaN-poisoned slots that
must never be read, sentinels around caller-owned outputs.  Where outputs are
bf16, values are scaled so |out| < 2, where bf16's own rounding is at most
2^-8 and the bar measures the kernel rather than the output format.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd._decode import group_tile, uses_gqa_kernel, valu_pair
from harness import (assert_parity, attention, decode_attention, kernel_args, max_err, oracle_attention, problem,
                     seeded)

pytestmark = pytest.mark.gpu


def _i32(values, device):
    return torch.tensor(values, device=device, dtype=torch.int32)


def _paged_pool(lengths, page, kv_heads, dim, dtype, device, seed, spare_cols=1, dim_v=None, scale=1.0):
    """K/V pages of a permuted pool; every slot past a request's length is NaN."""
    g = torch.Generator().manual_seed(seed)
    cols = max(-(-n // page) for n in lengths) + spare_cols
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols)
    kc = torch.randn(pool, page, kv_heads, dim, generator=g) * scale
    vc = torch.randn(pool, page, kv_heads, dim_v or dim, generator=g) * scale
    for b, n in enumerate(lengths):
        for pos in range(n, cols * page):
            kc[table[b, pos // page], pos % page] = float("nan")
            vc[table[b, pos // page], pos % page] = float("nan")
    return kc.to(dtype).to(device), vc.to(dtype).to(device), table.to(device), cols


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dqk,dv", [(64, 64), (128, 128), (256, 256), (96, 128), (192, 128)])
def test_packed_requests_of_0_to_513_keys(device, dtype, dqk, dv):
    """Five requests, one without a query, keys 0 / 1 / 256 / 513 / 257
    (test_decode.py:8-20)."""
    q = seeded((4, 6, dqk), 500 + dqk, dtype, device)
    k = seeded((1027, 2, dqk), 501 + dqk, dtype, device)
    v = seeded((1027, 2, dv), 502 + dv, dtype, device)
    cu_q, cu_k = _i32([0, 1, 2, 2, 3, 4], device), _i32([0, 0, 1, 257, 770, 1027], device)
    got, lse = decode_attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_k=513)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("splits", [1, 3, 16, 32])
@pytest.mark.parametrize("page", [16, 31, 256])
def test_paged_leftpad_views_and_poisoned_tails(device, splits, page):
    """K/V as stride-2 views of one [pages, heads, P, 512] buffer, left
    padding, NaN past every sequence, output into a strided sentinel view
    (test_decode.py:23-50: lengths 0 / 255 / 513, pads 3 / 7 / 1)."""
    lengths, pads = [0, 255, 513], [3, 7, 1]
    cols = -(-(max(lengths) + max(pads)) // page)
    g = torch.Generator().manual_seed(510 + page)
    table = torch.randperm(3 * cols, generator=g).int().reshape(3, cols).to(device)
    raw = seeded((3 * cols + 2, 2, page, 512), 511 + page, torch.float16, device)
    k, v = raw[1:-1].transpose(1, 2)[..., ::2].split(128, dim=-1)
    for b, (n, pad) in enumerate(zip(lengths, pads)):
        for pos in range(pad + n, cols * page):
            k[int(table[b, pos // page]), pos % page] = float("nan")
            v[int(table[b, pos // page]), pos % page] = float("nan")
    q = seeded((5, 8, 256), 512, torch.float16, device)[1:4, :, ::2]
    cu_q, used, left = _i32([0, 1, 2, 3], device), _i32(lengths, device), _i32(pads, device)
    buffer = torch.full((5, 8, 256), 123.0, device=device, dtype=torch.float16)
    out = buffer[1:4, :, ::2]
    got, lse = decode_attention(q, k, v, cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_k=513, block_table=table,
                                leftpad_k=left, num_splits=splits, out=out)
    assert got.data_ptr() == out.data_ptr()
    ref, ref_lse = oracle_attention(q, k, v, cu_q, used_k=used, block_table=table, leftpad=pads)
    assert_parity(got, lse, ref, ref_lse)
    assert (buffer[0] == 123).all() and (buffer[4] == 123).all() and (buffer[:, :, 1::2] == 123).all()


@pytest.mark.parametrize("splits", [0, 1, 5])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_page_walk_over_poisoned_pools(device, splits, kv_dtype):
    """The decode kernel's own layout (contiguous 16-token pages, 8/2 heads,
    d128), lengths 0 to 1029, fp32 output, FP8 with descales."""
    lengths = [1, 17, 300, 1029, 0, 64]
    kc, vc, table, _ = _paged_pool(lengths, 16, 2, 128, kv_dtype, device, seed=520)
    q = seeded((len(lengths), 8, 128), 521, torch.bfloat16, device)
    cu_q, used = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32), _i32(lengths, device)
    descale = torch.tensor([[0.5, 0.25]], device=device).expand(len(lengths), 2) if kv_dtype != torch.bfloat16 else None
    out = torch.empty(len(lengths), 8, 128, device=device, dtype=torch.float32)
    got, lse = decode_attention(q, kc, vc, cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_k=max(lengths),
                                block_table=table, num_splits=splits, out=out, k_descale=descale, v_descale=descale)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, k_descale=descale,
                                    v_descale=descale)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("heads,kv_heads", [(1, 1), (16, 1), (16, 8), (8, 8), (32, 8), (4, 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_query_head_groups_and_explicit_scale(device, heads, kv_heads, dtype):
    """MHA, MQA and GQA groups with softmax_scale 1/8 and 8 splits
    (test_decode.py:53-63: keys 3 and 257)."""
    q = seeded((2, heads, 128), 530 + heads, dtype, device)
    k = seeded((260, kv_heads, 128), 531 + kv_heads, dtype, device)
    v = seeded((260, kv_heads, 128), 532, dtype, device, scale=0.5)
    cu_q, cu_k = _i32([0, 1, 2], device), _i32([0, 3, 260], device)
    got, lse = decode_attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_k=257, softmax_scale=0.125,
                                num_splits=8)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, scale=0.125)
    assert_parity(got, lse, ref, ref_lse)


def test_no_queries_and_no_keys(device):
    """Zero query rows; then queries over zero keys (test_decode.py:66-76)."""
    q = torch.empty(0, 4, 128, device=device, dtype=torch.float16)
    k = torch.empty(0, 2, 128, device=device, dtype=torch.float16)
    zeros = _i32([0, 0, 0], device)
    got, lse = decode_attention(q, k, k, cu_seqlens_q=zeros, cu_seqlens_k=zeros, max_seqlen_k=0)
    assert got.shape == (0, 4, 128) and lse.shape == (4, 0)
    q = seeded((2, 4, 128), 540, torch.float16, device)
    got, lse = decode_attention(q, k, k, cu_seqlens_q=_i32([0, 1, 2], device), cu_seqlens_k=zeros, max_seqlen_k=0,
                                num_splits=4)
    assert torch.count_nonzero(got) == 0 and torch.isneginf(lse).all()


@pytest.mark.parametrize("q_dtype,k_dtype,v_dtype", [
    (torch.float16, torch.float8_e4m3fn, torch.float8_e4m3fn),
    (torch.float8_e4m3fn, torch.float8_e4m3fn, torch.float8_e4m3fn),
    (torch.float32, torch.bfloat16, torch.float16),
    (torch.bfloat16, torch.float8_e4m3fn, torch.float32),
    (torch.float16, torch.bfloat16, torch.float32),
])
def test_mixed_element_types_with_broadcast_descales(device, q_dtype, k_dtype, v_dtype):
    """Query, key and value of independent types, descales as stride-0
    expansions (test_decode.py:84-105); FP8 queries give fp16 output."""
    q = seeded((3, 8, 128), 550, q_dtype, device)
    k = seeded((261, 2, 128), 551, k_dtype, device)
    v = seeded((261, 2, 128), 552, v_dtype, device)
    cu_q, cu_k = _i32([0, 1, 2, 3], device), _i32([0, 1, 4, 261], device)
    qd = torch.tensor([[0.5], [0.75], [1.0]], device=device).expand(3, 2)
    kd = torch.tensor([[0.4, 0.6]], device=device).expand(3, 2)
    vd = torch.tensor([[0.2, 0.9]], device=device).expand(3, 2)
    got, lse = decode_attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_k=257, q_descale=qd,
                                k_descale=kd, v_descale=vd)
    assert got.dtype == (torch.float16 if q_dtype == torch.float8_e4m3fn else q_dtype)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, q_descale=qd, k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("window", [(-1, -1), (0, 0), (15, 0), (63, -1)])
@pytest.mark.parametrize("splits", [0, 1, 4])
def test_fp8_pages_with_sinks_windows_and_softcap(device, window, splits):
    """FP8 K/V halves of one [25, 16, 2, 256] pool whose last page is NaN
    and fills every unused table entry; sinks, softcap 0.7, descales, left
    padding, fp32 output (test_decode.py:108-133)."""
    raw = seeded((25, 16, 2, 256), 560, torch.float32, "cpu")
    raw[24] = float("nan")
    k, v = raw.to(torch.float8_e4m3fn).to(device).split(128, dim=-1)
    q = seeded((3, 8, 128), 561, torch.float16, device)
    cu_q, used, left = _i32([0, 1, 2, 3], device), _i32([0, 33, 97], device), _i32([0, 3, 1], device)
    table = _i32([[24] * 8, [3, 8, 11, 24, 24, 24, 24, 24], [4, 10, 7, 6, 2, 13, 21, 24]], device)
    qd = torch.tensor([[1.0, 0.75]], device=device).expand(3, 2)
    kd = torch.tensor([[0.5]], device=device).expand(3, 2)
    vd = torch.tensor([[0.25, 1.0]], device=device).expand(3, 2)
    sinks = torch.linspace(-3, 3, 16, device=device, dtype=torch.float16)[::2]
    out = torch.empty(3, 8, 128, device=device, dtype=torch.float32)
    got, lse = decode_attention(q, k, v, cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_k=97, block_table=table,
                                leftpad_k=left, num_splits=splits, window_size=window, softcap=0.7, q_descale=qd,
                                k_descale=kd, v_descale=vd, s_aux=sinks, out=out)
    assert got.data_ptr() == out.data_ptr()
    ref, ref_lse = oracle_attention(q, k, v, cu_q, used_k=used, block_table=table, leftpad=[0, 3, 1], q_descale=qd,
                                    k_descale=kd, v_descale=vd, sinks=sinks, softcap=0.7, window=window)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("splits", [1, 8])
def test_sinks_alone_when_there_are_no_keys(device, splits):
    """With no keys the LSE is the sink logit, counted once across splits
    (test_decode.py:136-146)."""
    q = seeded((2, 16, 128), 570, torch.float16, device)
    k = torch.empty(0, 8, 128, device=device, dtype=torch.float16)
    sinks = torch.linspace(-5, 5, 16, device=device)
    got, lse = decode_attention(q, k, k, cu_seqlens_q=_i32([0, 1, 2], device), cu_seqlens_k=_i32([0, 0, 0], device),
                                max_seqlen_k=0, num_splits=splits, s_aux=sinks, softcap=0.5)
    assert torch.count_nonzero(got) == 0
    assert max_err(lse, sinks[:, None].expand(16, 2)) <= 1e-6


def test_growing_context_and_split_counts_above_32(device):
    """Contexts 513 / 769 / 1025, then 33 / 65 / 129 splits of 1025 keys
    (test_decode.py:149-170)."""
    q = seeded((1, 4, 128), 580, torch.float16, device)
    k = seeded((1025, 2, 128), 581, torch.float16, device)
    v = seeded((1025, 2, 128), 582, torch.float16, device)
    cu_q = _i32([0, 1], device)
    for length in (513, 769, 1025):
        cu_k = _i32([0, length], device)
        got, lse = decode_attention(q, k[:length], v[:length], cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                                    max_seqlen_k=length)
        ref, ref_lse = oracle_attention(q, k[:length], v[:length], cu_q, cu_k)
        assert_parity(got, lse, ref, ref_lse, what=f"{length} keys")
    for splits in (33, 65, 129):
        got, lse = decode_attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_k=1025,
                                    num_splits=splits)
        assert_parity(got, lse, ref, ref_lse, what=f"{splits} splits")


def test_kernel_choice_does_not_depend_on_lengths(device):
    """Whether the decode kernel runs depends on types, dims and strides only
    (the reference pins no recompilation as lengths grow, test_decode.py:149-170)."""
    q = seeded((1, 4, 128), 590, torch.bfloat16, device)
    k = seeded((2048, 2, 128), 591, torch.bfloat16, device)
    out = torch.empty(1, 4, 128, device=device, dtype=torch.bfloat16)
    lse = torch.empty(4, 1, device=device)
    verdicts = set()
    for length in (1, 100, 2048):
        keep = []
        a = kernel_args(q, k, k, out, lse, keep=keep, cu_seqlens_q=_i32([0, 1], device),
                        cu_seqlens_k=_i32([0, length], device), max_seqlen_q=1, max_seqlen_k=length)
        verdicts.add(_lib.supported("fa_decode_supported", a))
    assert verdicts == {True}


@pytest.mark.parametrize("d", [32, 72, 80, 96])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("splits", [0, 3])
def test_head_dims_padded_inside_wider_tiles(device, d, kv_dtype, splits):
    """Head dims 32 and 72/80/96 run in the 64/128-wide tiles: the caches are
    views into NaN-filled 128-wide storage (a read past d poisons the result)
    and out's extra columns must stay untouched."""
    lengths, page, kv_heads, heads, width = [1, 40, 777, 0, 1500], 16, 2, 8, 128
    g = torch.Generator().manual_seed(600 + d + splits)
    cols = max(-(-n // page) for n in lengths) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols).to(device)
    q_dtype = torch.float16 if kv_dtype == torch.float16 else torch.bfloat16
    k_store = torch.full((pool, page, kv_heads, width), float("nan")).to(kv_dtype).to(device)
    v_store = torch.full((pool, page, kv_heads, width), float("nan")).to(kv_dtype).to(device)
    kc, vc = k_store[..., :d], v_store[..., :d]
    kc.copy_(torch.randn(pool, page, kv_heads, d, generator=g).to(kv_dtype))
    vc.copy_(torch.randn(pool, page, kv_heads, d, generator=g).to(kv_dtype))
    q = torch.randn(len(lengths), heads, d, generator=g).to(q_dtype).to(device)
    cu_q, used = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32), _i32(lengths, device)
    out_store = torch.full((len(lengths), heads, width), 7.0, device=device)
    out = out_store[..., :d]
    descale = (torch.tensor([[0.5, 0.25]], device=device).expand(len(lengths), 2)
               if kv_dtype == torch.float8_e4m3fn else None)
    keep = []
    probe = kernel_args(q, kc, vc, out, torch.empty(heads, len(lengths), device=device), keep=keep,
                        cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_q=1, max_seqlen_k=max(lengths),
                        block_table=table, k_descale=descale, v_descale=descale)
    assert _lib.supported("fa_decode_supported", probe)
    got, lse = decode_attention(q, kc, vc, cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_k=max(lengths),
                                block_table=table, num_splits=splits, out=out, k_descale=descale, v_descale=descale)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, k_descale=descale,
                                    v_descale=descale)
    assert_parity(got, lse, ref, ref_lse)
    assert (out_store[..., d:] == 7.0).all()


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("heads,kv_heads,d,tile", [(64, 8, 128, 8), (32, 2, 80, 8), (40, 8, 128, 8),
                                                   (28, 4, 96, 8), (12, 2, 128, 8), (14, 2, 64, 4),
                                                   (10, 2, 64, 4), (24, 8, 128, 4)])
@pytest.mark.parametrize("splits", [0, 1])
def test_query_head_tiles(device, kv_dtype, heads, kv_heads, d, tile, splits):
    """`tile` query heads of one KV head per workgroup (8 for 128-wide tiles,
    4 for 64-wide); groups of 16 take two workgroups, groups of 5-7 end in a
    partial tile whose spare slots must store nothing.  Spare table entries
    point at a NaN page; sinks, softcap 20, FP8 descales.  Pages of 8 tokens
    keep these groups on the VALU kernel (the matrix-core decode needs pages
    of a multiple of 16)."""
    assert group_tile(heads, kv_heads, d, d) == tile
    lengths, page = [1, 300, 2049, 0, 77], 8
    g = torch.Generator().manual_seed(610 + heads + d + splits)
    cols = max(-(-n // page) for n in lengths) + 1
    pool = len(lengths) * cols + 1
    table = torch.randperm(pool - 1, generator=g)[: len(lengths) * cols].int().reshape(len(lengths), cols)
    table[:, -1] = pool - 1
    scale = 0.5 if kv_dtype == torch.bfloat16 else 1.0
    kc = torch.randn(pool, page, kv_heads, d, generator=g)
    vc = torch.randn(pool, page, kv_heads, d, generator=g) * scale
    kc[pool - 1] = vc[pool - 1] = float("nan")
    kc, vc = kc.to(kv_dtype).to(device), vc.to(kv_dtype).to(device)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cu_q, used, table = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32), _i32(lengths, device), table.to(device)
    sinks = torch.linspace(-2, 2, heads, device=device)
    fp8 = kv_dtype == torch.float8_e4m3fn
    kd = (torch.rand(len(lengths), kv_heads, generator=g) * 0.5 + 0.5).to(device) if fp8 else None
    vd = (torch.rand(len(lengths), kv_heads, generator=g) * 0.25 + 0.25).to(device) if fp8 else None
    buffer = torch.full((len(lengths), heads + 8, d), 7.0, device=device, dtype=torch.bfloat16)
    got, lse = decode_attention(q, kc, vc, cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_k=cols * page,
                                block_table=table, num_splits=splits, softcap=20.0, s_aux=sinks, k_descale=kd,
                                v_descale=vd, out=buffer[:, :heads])
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, sinks=sinks, softcap=20.0,
                                    k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)
    assert (buffer[:, heads:] == 7.0).all(), "a spare head slot was stored"


@pytest.mark.parametrize("heads,kv_heads,d", [(32, 8, 128), (40, 8, 128), (14, 2, 64), (16, 8, 256)])
@pytest.mark.parametrize("per_request", [False, True])
@pytest.mark.parametrize("splits", [0, 1])
def test_alibi_on_the_decode_kernel(device, heads, kv_heads, d, per_request, splits):
    """ALiBi slopes [Hq] or [B, Hq] through the router: the single query sits
    at key k_len - 1, so key j is biased by -slope (k_len - 1 - j); with left
    padding, a left window, sinks and split counts."""
    lengths, left, page = [1, 300, 2049, 0, 77], [0, 5, 0, 0, 3], 16
    stored = [n + p for n, p in zip(lengths, left)]      # padding, then the visible keys
    kc, vc, table, cols = _paged_pool(stored, page, kv_heads, d, torch.bfloat16, device, seed=620 + heads + d)
    vc = vc * 0.5
    g = torch.Generator().manual_seed(621 + per_request)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cu_q = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32)
    used, pads = _i32(lengths, device), _i32(left, device)
    slopes = (torch.rand((len(lengths), heads) if per_request else (heads,), generator=g) * 0.2).to(device)
    sinks = torch.linspace(-1, 1, heads, device=device)
    kw = dict(cu_seqlens_q=cu_q, seqused_k=used, max_seqlen_q=1, max_seqlen_k=cols * page, block_table=table,
              alibi_slopes=slopes, window_size=(1000, 0), s_aux=sinks, leftpad_k=pads)
    keep = []
    probe = kernel_args(q, kc, vc, torch.empty_like(q), torch.empty(heads, len(lengths), device=device), keep=keep,
                        **kw)
    assert _lib.supported("fa_decode_supported", probe)
    got, lse = attention(q, kc, vc, causal=True, num_splits=splits, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, leftpad=left, alibi=slopes,
                                    window=(1000, 0), sinks=sinks)
    assert_parity(got, lse, ref, ref_lse)


def _padded_pool(lengths, left, page, kv_heads, width_k, width_v, dtype, seed, scale_v=1.0):
    """Paged K/V of a permuted pool with K / V rows of width_k / width_v
    elements per head; slot j of request b is real for left[b] <= j <
    left[b] + lengths[b] and NaN elsewhere (left padding and tails)."""
    g = torch.Generator().manual_seed(seed)
    stored = [n + p for n, p in zip(lengths, left)]
    cols = max(-(-n // page) for n in stored) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols)
    kc = torch.randn(pool, page, kv_heads, width_k, generator=g)
    vc = torch.randn(pool, page, kv_heads, width_v, generator=g) * scale_v
    for b, n in enumerate(stored):
        for pos in list(range(0, left[b])) + list(range(n, cols * page)):
            kc[table[b, pos // page], pos % page] = float("nan")
            vc[table[b, pos // page], pos % page] = float("nan")
    return kc.to(dtype), vc.to(dtype), table, cols, g


def _pair_case(device, kv_dtype, dq, dv, heads, kv_heads, splits, page, window, stride_mult, seed):
    """One decode call with sinks, softcap 30, per-(request, KV head) k/v
    descales, NaN left padding and tails; heads sliced from rows
    `stride_mult` times their width.  Returns (problem, got, reference)."""
    lengths, left = [1, 31, 300, 0, 2049, 77], [0, 3, 17, 0, 5, 16]
    fp8 = kv_dtype == torch.float8_e4m3fn
    kc, vc, table, cols, g = _padded_pool(lengths, left, page, kv_heads, stride_mult * dq, stride_mult * dv, kv_dtype,
                                          seed, 1.0 if fp8 else 0.5)
    q_dtype = torch.float16 if kv_dtype == torch.float16 else torch.bfloat16
    q = torch.randn(len(lengths), heads, dq, generator=g).to(q_dtype)
    kd = torch.rand(len(lengths), kv_heads, generator=g) * (0.1 if fp8 else 0.5) + (0.05 if fp8 else 0.75)
    vd = torch.rand(len(lengths), kv_heads, generator=g) * 0.5 + 0.25
    sinks = torch.linspace(-2, 2, heads)
    cu_q, used, pads = (torch.arange(len(lengths) + 1, dtype=torch.int32), torch.tensor(lengths, dtype=torch.int32),
                        torch.tensor(left, dtype=torch.int32))
    kg, vg = kc.to(device)[..., :dq], vc.to(device)[..., :dv]
    kw = dict(cu_seqlens_q=cu_q.to(device), seqused_k=used.to(device), block_table=table.to(device),
              leftpad_k=pads.to(device), window_size=window, softcap=30.0, s_aux=sinks.to(device),
              k_descale=kd.to(device), v_descale=vd.to(device))
    p = problem(q.to(device), kg, vg, max_seqlen_q=1, max_seqlen_k=cols * page, **kw)
    got, lse = decode_attention(q.to(device), kg, vg, max_seqlen_k=cols * page, num_splits=splits, **kw)
    ref, ref_lse = oracle_attention(q, kc[..., :dq], vc[..., :dv], cu_q, used_k=used, block_table=table, leftpad=left,
                                    window=window, softcap=30.0, sinks=sinks, k_descale=kd, v_descale=vd)
    return p, (got, lse), (ref, ref_lse)


@pytest.mark.parametrize("kv_dtype,dq,dv,heads,kv_heads", [
    (torch.float8_e4m3fn, 128, 128, 8, 8), (torch.float8_e4m3fn, 128, 128, 16, 8),
    (torch.float8_e4m3fn, 128, 128, 32, 16), (torch.bfloat16, 192, 128, 8, 8), (torch.float16, 192, 128, 16, 16)])
@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("page,window", [(16, (-1, -1)), (8, (700, 0))])
def test_paired_kv_heads(device, kv_dtype, dq, dv, heads, kv_heads, splits, page, window):
    """Two neighbouring KV heads per workgroup, each lane loading its pieces
    of both heads' rows: per-(request, KV head) k/v descales that differ
    between the heads of a pair (a query head scaled with its neighbour's
    descale fails the bar), sinks, softcap 30, a left window, NaN left
    padding and tails."""
    p, (got, lse), (ref, ref_lse) = _pair_case(device, kv_dtype, dq, dv, heads, kv_heads, splits, page, window, 1,
                                               880 + dq + heads + splits + page)
    assert not uses_gqa_kernel(p) and valu_pair(p) == 2
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("case", ["strided", "few", "wide_rows", "group"])
def test_unpaired_kv_head_layouts(device, case):
    """One KV head per workgroup: heads sliced from wider rows (head stride
    2 d), fewer than 8 KV heads, 256-byte head rows (16-bit d128), and
    192/128 groups of 2."""
    kv_dtype, dq, dv, heads, kv_heads, mult = {
        "strided": (torch.float8_e4m3fn, 128, 128, 16, 8, 2), "few": (torch.float8_e4m3fn, 128, 128, 8, 4, 1),
        "wide_rows": (torch.bfloat16, 128, 128, 16, 8, 1), "group": (torch.bfloat16, 192, 128, 16, 8, 1)}[case]
    p, (got, lse), (ref, ref_lse) = _pair_case(device, kv_dtype, dq, dv, heads, kv_heads, 3, 16, (-1, -1), mult,
                                               890 + len(case))
    assert not uses_gqa_kernel(p) and valu_pair(p) == 1
    assert_parity(got, lse, ref, ref_lse)
