"""Split-KV decode on gfx950 vs the fp64 oracle.

Ports flash_attn_mps tests/test_decode.py:8-174: packed dims, paged +
leftpad + strided views + poisoned tails for several split counts and page
sizes, GQA/MQA, empty queries/KV, independent dtypes with broadcast
descales, paged FP8 with sinks/windows/softcap, sinks counted once, growing
KV and large split counts; query-head groups of 4 to 16 per KV head,
including groups the head tile does not divide; ALiBi slopes.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd._decode import decode_attention
from helpers import assert_attention_close, attention_reference

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dims", [(64, 64), (128, 128), (256, 256), (96, 128), (192, 128)])
def test_decode_packed_against_fp64(device, dtype, dims):
    dq, dv = dims
    q = torch.randn(4, 6, dq, device=device, dtype=dtype)
    k = torch.randn(1027, 2, dq, device=device, dtype=dtype)
    v = torch.randn(1027, 2, dv, device=device, dtype=dtype)
    cq = torch.tensor([0, 1, 2, 2, 3, 4], device=device, dtype=torch.int32)
    ck = torch.tensor([0, 0, 1, 257, 770, 1027], device=device, dtype=torch.int32)
    actual, lse = decode_attention(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck, max_seqlen_k=513)
    expected, el = attention_reference(q, k, v, cq, ck)
    assert_attention_close(actual, expected, dtype)
    torch.testing.assert_close(lse.cpu().double(), el, atol=8e-6, rtol=2e-5)


@pytest.mark.parametrize("splits", [1, 3, 16, 32])
@pytest.mark.parametrize("page", [16, 31, 256])
def test_decode_paged_leftpad_strides_and_partial_tail(device, splits, page):
    lengths = [0, 255, 513]
    pads = [3, 7, 1]
    columns = (max(lengths) + max(pads) + page - 1) // page
    table = torch.randperm(3 * columns, device=device).int().reshape(3, columns)
    # Shared K/V storage views with unequal token/head strides, a non-unit
    # head-dim stride and a nonzero storage offset.
    raw = torch.randn(3 * columns + 2, 2, page, 512, device=device, dtype=torch.float16)
    k, v = raw[1:-1].transpose(1, 2)[..., ::2].split(128, dim=-1)
    for b, (length, pad) in enumerate(zip(lengths, pads)):
        for pos in range(pad + length, columns * page):
            physical = int(table[b, pos // page])
            k[physical, pos % page] = float("nan")
            v[physical, pos % page] = float("nan")
    q = torch.randn(5, 8, 256, device=device, dtype=torch.float16)[1:4, :, ::2]
    cq = torch.tensor([0, 1, 2, 3], device=device, dtype=torch.int32)
    used = torch.tensor(lengths, device=device, dtype=torch.int32)
    left = torch.tensor(pads, device=device, dtype=torch.int32)
    out_storage = torch.full((5, 8, 256), 123., device=device, dtype=torch.float16)
    out = out_storage[1:4, :, ::2]
    actual, lse = decode_attention(q, k, v, cu_seqlens_q=cq, seqused_k=used, max_seqlen_k=513,
                                   block_table=table, leftpad_k=left, num_splits=splits, out=out)
    expected, el = attention_reference(q, k, v, cq, used_k=used, block_table=table, leftpad=pads)
    assert actual.data_ptr() == out.data_ptr()
    assert_attention_close(actual, expected)
    torch.testing.assert_close(lse.cpu().double(), el, atol=8e-6, rtol=2e-5)
    assert torch.all(out_storage[0] == 123) and torch.all(out_storage[4] == 123)
    assert torch.all(out_storage[:, :, 1::2] == 123)


@pytest.mark.parametrize("splits", [0, 1, 5])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_decode_fast_path_paged_contiguous_poisoned(device, splits, dtype):
    """The gfx950 decode kernel itself (contiguous 16-token pages): poisoned
    unused slots must never be read."""
    g = torch.Generator().manual_seed(5)
    lengths = [1, 17, 300, 1029, 0, 64]
    page, hkv, heads, d = 16, 2, 8, 128
    cols = max((n + page - 1) // page for n in lengths) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols)
    kc = torch.randn(pool, page, hkv, d, generator=g)
    vc = torch.randn(pool, page, hkv, d, generator=g)
    for b, n in enumerate(lengths):
        for pos in range(n, cols * page):
            kc[table[b, pos // page], pos % page] = float("nan")
            vc[table[b, pos // page], pos % page] = float("nan")
    kc, vc = kc.to(dtype).to(device), vc.to(dtype).to(device)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cq = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32)
    used = torch.tensor(lengths, device=device, dtype=torch.int32)
    table = table.to(device)
    out = torch.empty(len(lengths), heads, d, device=device, dtype=torch.float32)
    kd = torch.tensor([[0.5, 0.25]], device=device).expand(len(lengths), 2) if dtype != torch.bfloat16 else None
    args_ok = True
    actual, lse = decode_attention(q, kc, vc, cu_seqlens_q=cq, seqused_k=used, max_seqlen_k=max(lengths),
                                   block_table=table, num_splits=splits, out=out, k_descale=kd, v_descale=kd)
    expected, el = attention_reference(q, kc, vc, cq, used_k=used, block_table=table, k_descale=kd, v_descale=kd)
    assert args_ok
    torch.testing.assert_close(actual.cpu().double(), expected, atol=2e-5, rtol=2e-4)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-5, rtol=2e-5)


@pytest.mark.parametrize("heads,kvheads", [(1, 1), (16, 1), (16, 8), (8, 8)])
def test_decode_gqa_mqa_and_scaling(device, heads, kvheads):
    q = torch.randn(2, heads, 128, device=device, dtype=torch.float32)
    k = torch.randn(260, kvheads, 128, device=device, dtype=torch.float32)
    v = torch.randn_like(k)
    cq = torch.tensor([0, 1, 2], device=device, dtype=torch.int32)
    ck = torch.tensor([0, 3, 260], device=device, dtype=torch.int32)
    actual, lse = decode_attention(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck,
                                   max_seqlen_k=257, softmax_scale=.125, num_splits=8)
    expected, el = attention_reference(q, k, v, cq, ck, scale=.125)
    torch.testing.assert_close(actual.cpu().double(), expected, atol=8e-6, rtol=2e-4)
    torch.testing.assert_close(lse.cpu().double(), el, atol=8e-6, rtol=2e-5)


@pytest.mark.parametrize("heads,kvheads", [(32, 8), (16, 1), (4, 2)])
def test_decode_gqa_bf16_fast_kernel(device, heads, kvheads):
    q = torch.randn(3, heads, 128, device=device, dtype=torch.bfloat16)
    k = torch.randn(900, kvheads, 128, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    cq = torch.tensor([0, 1, 2, 3], device=device, dtype=torch.int32)
    ck = torch.tensor([0, 3, 260, 900], device=device, dtype=torch.int32)
    actual, lse = decode_attention(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck, max_seqlen_k=640)
    expected, el = attention_reference(q, k, v, cq, ck)
    assert_attention_close(actual, expected, torch.bfloat16)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-5, rtol=2e-5)


def test_decode_empty_queries_and_kv(device):
    q = torch.empty(0, 4, 128, device=device, dtype=torch.float16)
    k = torch.empty(0, 2, 128, device=device, dtype=torch.float16)
    cq = torch.tensor([0, 0, 0], device=device, dtype=torch.int32)
    result, lse = decode_attention(q, k, k, cu_seqlens_q=cq, cu_seqlens_k=cq, max_seqlen_k=0)
    assert result.shape == (0, 4, 128) and lse.shape == (4, 0)
    q = torch.randn(2, 4, 128, device=device, dtype=torch.float16)
    result, lse = decode_attention(q, k, k, cu_seqlens_q=torch.tensor([0, 1, 2], device=device, dtype=torch.int32),
                                   cu_seqlens_k=cq, max_seqlen_k=0, num_splits=4)
    assert torch.count_nonzero(result) == 0
    assert torch.isneginf(lse).all()


def _typed_random(shape, dtype, device):
    return torch.randn(shape).to(dtype).to(device)


@pytest.mark.parametrize("dtypes", [
    (torch.float16, torch.float8_e4m3fn, torch.float8_e4m3fn),
    (torch.float8_e4m3fn, torch.float8_e4m3fn, torch.float8_e4m3fn),
    (torch.float32, torch.bfloat16, torch.float16),
    (torch.bfloat16, torch.float8_e4m3fn, torch.float32),
    (torch.float16, torch.bfloat16, torch.float32),
])
def test_decode_independent_dtypes_and_broadcast_descales(device, dtypes):
    q = _typed_random((3, 8, 128), dtypes[0], device)
    k = _typed_random((261, 2, 128), dtypes[1], device)
    v = _typed_random((261, 2, 128), dtypes[2], device)
    cq = torch.tensor([0, 1, 2, 3], device=device, dtype=torch.int32)
    ck = torch.tensor([0, 1, 4, 261], device=device, dtype=torch.int32)
    qs = torch.tensor([[.5], [.75], [1.]], device=device).expand(3, 2)
    ks = torch.tensor([[.4, .6]], device=device).expand(3, 2)
    vs = torch.tensor([[.2, .9]], device=device).expand(3, 2)
    out, lse = decode_attention(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck, max_seqlen_k=257,
                                q_descale=qs, k_descale=ks, v_descale=vs)
    expected, el = attention_reference(q, k, v, cq, ck, q_descale=qs, k_descale=ks, v_descale=vs)
    assert out.dtype == (torch.float16 if dtypes[0] == torch.float8_e4m3fn else dtypes[0])
    assert_attention_close(out, expected, out.dtype)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-5, rtol=2e-5)


@pytest.mark.parametrize("window", [(-1, -1), (0, 0), (15, 0), (63, -1)])
@pytest.mark.parametrize("splits", [0, 1, 4])
def test_decode_paged_fp8_sink_window_and_softcap(device, window, splits):
    raw = torch.randn(25, 16, 2, 256)
    raw[24] = float("nan")   # unused page-table entries point at this poisoned page
    packed = raw.to(torch.float8_e4m3fn).to(device)
    k, v = packed.split(128, dim=-1)
    q = _typed_random((3, 8, 128), torch.float16, device)
    cq = torch.tensor([0, 1, 2, 3], device=device, dtype=torch.int32)
    used = torch.tensor([0, 33, 97], device=device, dtype=torch.int32)
    left = torch.tensor([0, 3, 1], device=device, dtype=torch.int32)
    table = torch.tensor([[24] * 8, [3, 8, 11, 24, 24, 24, 24, 24],
                          [4, 10, 7, 6, 2, 13, 21, 24]], device=device, dtype=torch.int32)
    qs = torch.tensor([[1., .75]], device=device).expand(3, 2)
    ks = torch.tensor([[.5]], device=device).expand(3, 2)
    vs = torch.tensor([[.25, 1.]], device=device).expand(3, 2)
    sinks = torch.linspace(-3, 3, 16, device=device, dtype=torch.float16)[::2]
    output = torch.empty((3, 8, 128), device=device, dtype=torch.float32)
    out, lse = decode_attention(q, k, v, cu_seqlens_q=cq, seqused_k=used, max_seqlen_k=97,
                                block_table=table, leftpad_k=left, num_splits=splits, window_size=window,
                                softcap=.7, q_descale=qs, k_descale=ks, v_descale=vs, s_aux=sinks, out=output)
    expected, el = attention_reference(q, k, v, cq, used_k=used, block_table=table, leftpad=[0, 3, 1],
                                       q_descale=qs, k_descale=ks, v_descale=vs, sinks=sinks, softcap=.7,
                                       window=window)
    assert out.data_ptr() == output.data_ptr()
    torch.testing.assert_close(out.cpu().double(), expected, atol=8e-6, rtol=2e-4)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-5, rtol=2e-5)


@pytest.mark.parametrize("splits", [1, 8])
def test_decode_sinks_seed_empty_kv_only_once(device, splits):
    q = torch.randn(2, 16, 128, device=device, dtype=torch.float16)
    k = torch.empty(0, 8, 128, device=device, dtype=torch.float16)
    cq = torch.tensor([0, 1, 2], device=device, dtype=torch.int32)
    ck = torch.tensor([0, 0, 0], device=device, dtype=torch.int32)
    sinks = torch.linspace(-5, 5, 16, device=device)
    out, lse = decode_attention(q, k, k, cu_seqlens_q=cq, cu_seqlens_k=ck, max_seqlen_k=0,
                                num_splits=splits, s_aux=sinks, softcap=.5)
    assert torch.count_nonzero(out) == 0
    torch.testing.assert_close(lse, sinks[:, None].expand(16, 2), atol=1e-6, rtol=1e-6)


def test_decode_kv_growth_and_large_split_count(device):
    q = torch.randn(1, 4, 128, device=device, dtype=torch.float16)
    k = torch.randn(1025, 2, 128, device=device, dtype=torch.float16)
    v = torch.randn_like(k)
    cq = torch.tensor([0, 1], device=device, dtype=torch.int32)
    for length in (513, 769, 1025):
        ck = torch.tensor([0, length], device=device, dtype=torch.int32)
        actual, lse = decode_attention(q, k[:length], v[:length], cu_seqlens_q=cq,
                                       cu_seqlens_k=ck, max_seqlen_k=length)
        expected, el = attention_reference(q, k[:length], v[:length], cq, ck)
        assert_attention_close(actual, expected)
        torch.testing.assert_close(lse.cpu().double(), el, atol=1e-5, rtol=2e-5)
    for splits in (33, 65, 129):
        actual, lse = decode_attention(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck,
                                       max_seqlen_k=1025, num_splits=splits)
        assert_attention_close(actual, expected)
        torch.testing.assert_close(lse.cpu().double(), el, atol=1e-5, rtol=2e-5)


def test_decode_kernel_choice_ignores_lengths(device):
    """Kernel choice depends on dtypes/dims/strides only (the reference pins
    'no recompilation as lengths grow', test_decode.py:153-174)."""
    from flash_attn_mps_amd._attention import build_args
    q = torch.randn(1, 4, 128, device=device, dtype=torch.bfloat16)
    k = torch.randn(2048, 2, 128, device=device, dtype=torch.bfloat16)
    cq = torch.tensor([0, 1], device=device, dtype=torch.int32)
    choices = set()
    for length in (1, 100, 2048):
        ck = torch.tensor([0, length], device=device, dtype=torch.int32)
        out = torch.empty(1, 4, 128, device=device, dtype=torch.bfloat16)
        lse = torch.empty(4, 1, device=device)
        keep = []
        a = build_args(q, k, k, out, lse, cu_seqlens_q=cq, cu_seqlens_k=ck, seqused_k=None, max_seqlen_q=1,
                       max_seqlen_k=length, block_table=None, softmax_scale=None, causal=False,
                       window_size=(-1, -1), alibi_slopes=None, softcap=0., s_aux=None, q_descale=None,
                       k_descale=None, v_descale=None, mask_mod=None, aux_tensors=None, leftpad_k=None, keep=keep)
        choices.add(_lib.supported("fa_decode_supported", a))
    assert choices == {True}


@pytest.mark.parametrize("d", [32, 72, 80, 96])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("splits", [0, 3])
def test_decode_padded_head_dims(device, d, dtype, splits):
    """Head dims 32 and 72/80/96 run on the decode kernel in its 64/128-dim
    tiles.  The caches are views into wider NaN-filled storage, so any read
    past the head dim would poison the result; out's extra columns must stay
    untouched."""
    from flash_attn_mps_amd._attention import build_args
    g = torch.Generator().manual_seed(d * 3 + splits)
    lengths = [1, 40, 777, 0, 1500]
    page, hkv, heads, width = 16, 2, 8, 128
    cols = max((n + page - 1) // page for n in lengths) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols).to(device)
    qdt = torch.float16 if dtype == torch.float16 else torch.bfloat16
    kst = torch.full((pool, page, hkv, width), float("nan")).to(dtype).to(device)
    vst = torch.full((pool, page, hkv, width), float("nan")).to(dtype).to(device)
    kc, vc = kst[..., :d], vst[..., :d]
    kc.copy_(torch.randn(pool, page, hkv, d, generator=g).to(dtype))
    vc.copy_(torch.randn(pool, page, hkv, d, generator=g).to(dtype))
    q = torch.randn(len(lengths), heads, d, generator=g).to(qdt).to(device)
    cq = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32)
    used = torch.tensor(lengths, device=device, dtype=torch.int32)
    ost = torch.full((len(lengths), heads, width), 7.0, device=device, dtype=torch.float32)
    out = ost[..., :d]
    desc = torch.tensor([[0.5, 0.25]], device=device).expand(len(lengths), 2) if dtype == torch.float8_e4m3fn else None
    lse_buf = torch.empty(heads, len(lengths), device=device)
    keep = []
    args = build_args(q, kc, vc, out, lse_buf, cu_seqlens_q=cq, cu_seqlens_k=None, seqused_k=used, max_seqlen_q=1,
                      max_seqlen_k=max(lengths), block_table=table, softmax_scale=None, causal=True,
                      window_size=(-1, -1), alibi_slopes=None, softcap=0., s_aux=None, q_descale=None,
                      k_descale=desc, v_descale=desc, mask_mod=None, aux_tensors=None, leftpad_k=None, keep=keep)
    assert _lib.supported("fa_decode_supported", args)
    actual, lse = decode_attention(q, kc, vc, cu_seqlens_q=cq, seqused_k=used, max_seqlen_k=max(lengths),
                                   block_table=table, num_splits=splits, out=out, k_descale=desc, v_descale=desc)
    expected, el = attention_reference(q, kc, vc, cq, used_k=used, block_table=table, k_descale=desc, v_descale=desc)
    torch.testing.assert_close(actual.cpu().double(), expected, atol=2e-3 if qdt == torch.float16 else 1e-2, rtol=0)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-4, rtol=0)
    assert torch.all(ost[..., d:] == 7.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("heads,kvheads,d,gt", [(64, 8, 128, 8), (32, 2, 80, 8), (40, 8, 128, 8), (28, 4, 96, 8),
                                                (12, 2, 128, 8), (14, 2, 64, 4), (10, 2, 64, 4), (24, 8, 128, 4)])
@pytest.mark.parametrize("splits", [0, 1])
def test_decode_head_tiles(device, dtype, heads, kvheads, d, gt, splits):
    """GT query heads of one KV head per workgroup: 8 for 128-dim tiles and 4
    for 64-dim ones; groups of 16 take two workgroups, groups of 5, 6 or 7 end
    in a partial tile whose spare slots store nothing.  Paged, NaN-poisoned
    spare pages, sinks, softcap, FP8 descales, empty and single-key requests."""
    from flash_attn_mps_amd._decode import decode_group_tile
    assert decode_group_tile(heads, kvheads, d, d) == gt
    g = torch.Generator().manual_seed(heads + d + splits)
    lengths = [1, 300, 2049, 0, 77]
    page = 16
    cols = max((n + page - 1) // page for n in lengths) + 1
    pool = len(lengths) * cols + 1
    table = torch.randperm(pool - 1, generator=g)[:len(lengths) * cols].int().reshape(len(lengths), cols)
    table[:, -1] = pool - 1
    kc = torch.randn(pool, page, kvheads, d, generator=g)
    vc = torch.randn(pool, page, kvheads, d, generator=g)
    kc[pool - 1] = float("nan")
    vc[pool - 1] = float("nan")
    kc, vc = kc.to(dtype).to(device), vc.to(dtype).to(device)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cq = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32)
    used = torch.tensor(lengths, device=device, dtype=torch.int32)
    table = table.to(device)
    sinks = torch.linspace(-2, 2, heads, device=device)
    fp8 = dtype == torch.float8_e4m3fn
    ks = torch.rand(len(lengths), kvheads, generator=g).add(0.5).to(device) if fp8 else None
    vs = torch.rand(len(lengths), kvheads, generator=g).add(0.5).to(device) if fp8 else None
    storage = torch.full((len(lengths), heads + 8, d), 7.0, device=device, dtype=torch.bfloat16)
    out, lse = decode_attention(q, kc, vc, cu_seqlens_q=cq, seqused_k=used, max_seqlen_k=cols * page,
                                block_table=table, num_splits=splits, softcap=20.0, s_aux=sinks,
                                k_descale=ks, v_descale=vs, out=storage[:, :heads])
    expected, el = attention_reference(q, kc, vc, cq, used_k=used, block_table=table, sinks=sinks,
                                       softcap=20.0, k_descale=ks, v_descale=vs)
    assert_attention_close(out, expected, torch.bfloat16)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-4, rtol=2e-5)
    assert torch.all(storage[:, heads:] == 7.0), "a spare head slot was stored"


@pytest.mark.parametrize("heads,kvheads,d", [(32, 8, 128), (40, 8, 128), (14, 2, 64), (16, 8, 256)])
@pytest.mark.parametrize("per_request", [False, True])
@pytest.mark.parametrize("splits", [0, 1])
def test_decode_alibi(device, heads, kvheads, d, per_request, splits):
    """ALiBi on the decode kernel: the single query sits at key k_len - 1, so
    key j gets -slope (k_len - 1 - j); [Hq] or [B, Hq] slopes, with leftpad,
    a left window, sinks and split counts, through the public route
    (attention -> decode_attention).  ALiBi with softcap stays on the generic
    kernel."""
    from flash_attn_mps_amd._attention import attention, build_args
    g = torch.Generator().manual_seed(heads + d + per_request)
    lengths, left = [1, 300, 2049, 0, 77], [0, 5, 0, 0, 3]
    page = 16
    cols = max((n + page - 1) // page for n in lengths) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols).to(device)
    kc = torch.randn(pool, page, kvheads, d, generator=g).to(torch.bfloat16).to(device)
    vc = torch.randn(pool, page, kvheads, d, generator=g).to(torch.bfloat16).to(device)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cq = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32)
    used = torch.tensor([n + p for n, p in zip(lengths, left)], device=device, dtype=torch.int32)
    lp = torch.tensor(left, device=device, dtype=torch.int32)
    shape = (len(lengths), heads) if per_request else (heads,)
    slopes = (torch.rand(shape, generator=g) * 0.2).to(device)
    sinks = torch.linspace(-1, 1, heads, device=device)
    kw = dict(cu_seqlens_q=cq, seqused_k=used, max_seqlen_q=1, max_seqlen_k=cols * page, block_table=table,
              alibi_slopes=slopes, softcap=0.0, window_size=(1000, 0), s_aux=sinks, leftpad_k=lp,
              num_splits=splits)
    keep = []
    probe = build_args(q, kc, vc, torch.empty_like(q), torch.empty(heads, len(lengths), device=device), keep=keep,
                       causal=False, softmax_scale=None, q_descale=None, k_descale=None, v_descale=None,
                       mask_mod=None, aux_tensors=None, cu_seqlens_k=None,
                       **{k: v for k, v in kw.items() if k not in ("s_aux", "num_splits")}, s_aux=sinks)
    assert _lib.supported("fa_decode_supported", probe)
    out, lse = attention(q, kc, vc, causal=True, **kw)
    expected, el = attention_reference(q, kc, vc, cq, used_k=used, block_table=table, leftpad=left,
                                       alibi=slopes, window=(1000, 0), sinks=sinks)
    assert_attention_close(out, expected, torch.bfloat16)
    torch.testing.assert_close(lse.cpu().double(), el, atol=1e-4, rtol=2e-5)
