"""BASELINE configurations 1-5 at full size on the GPU vs the fp64 oracle.

Each configuration is generated exactly as bench.py generates it.  Config 1
is checked in full; configs 2-5 are too large for a CPU fp64 sweep of every
row, so the oracle recomputes sampled query rows (first, last and random rows
of every request, or sampled requests for decode), which is exact for those
rows because attention rows are independent.  Cache writes are checked
byte-for-byte against the oracle's scatter.
"""
import pytest
import torch

import bench
from flash_attn_mps_amd import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache, vllm
from helpers import assert_north_star, attention_reference, cu_from_lengths
from oracle import cache as ocache

pytestmark = pytest.mark.gpu


def _sample_rows(q_lens, per_request=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    rows, start = [], 0
    for n in q_lens:
        if n:
            picks = {0, n - 1} | set(torch.randint(0, n, (min(n, per_request),), generator=g).tolist())
            rows += [start + p for p in sorted(picks)]
        start += n
    return torch.tensor(rows, dtype=torch.long)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_config1_dense_causal_gqa(device, dtype):
    g = torch.Generator().manual_seed(123 + 1)
    q = torch.randn(2, 128, 16, 128, generator=g)
    k = torch.randn(2, 128, 8, 128, generator=g)
    v = torch.randn(2, 128, 8, 128, generator=g)
    q, k, v = (t.to(dtype) for t in (q, k, v))
    out, lse = flash_attn_func(q.to(device), k.to(device), v.to(device), softmax_scale=128 ** -0.5, causal=True,
                               return_softmax_lse=True)
    assert out.shape == (2, 128, 16, 128) and lse.shape == (2, 16, 128)
    cu = torch.tensor([0, 128, 256], dtype=torch.int32)
    ref, ref_lse = attention_reference(q.flatten(0, 1), k.flatten(0, 1), v.flatten(0, 1), cu, cu, causal=True)
    assert_north_star(out.flatten(0, 1), lse.transpose(0, 1).reshape(16, -1), ref, ref_lse, dtype)


def test_config2_varlen_causal_prefill_full_size(device):
    r = bench.config2(device, steps=1, warmup=0)
    q, k, v, cu = r["tensors"]
    lengths = r["lengths"]
    out, lse = flash_attn_varlen_func(q, k, v, cu, cu, max(lengths), max(lengths), causal=True,
                                      return_softmax_lse=True)
    rows = _sample_rows(lengths, seed=2)
    ref, ref_lse = attention_reference(q, k, v, cu, cu, causal=True, rows=rows)
    assert_north_star(out, lse, ref, ref_lse, torch.bfloat16, rows=rows)


def _gather_request(kc, vc, table, b, length, page):
    n = (length + page - 1) // page
    pages = table[b, :n].long()
    return kc[pages].cpu(), vc[pages].cpu(), torch.arange(n, dtype=torch.int32).reshape(1, n)


def test_config3_paged_decode_full_size(device):
    g = torch.Generator().manual_seed(123 + 3)
    ctx = torch.randint(512, 32769, (64,), generator=g).tolist()
    hq, hkv, d, page = 32, 8, 128, 16
    kc, vc, table, slots = bench.paged_cache(ctx, page, hkv, d, torch.bfloat16, device, 123 + 3)
    q = torch.randn(64, 1, hq, d, generator=g).to(torch.bfloat16).to(device)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    out, lse = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=lens, block_table=table, causal=True,
                                       return_softmax_lse=True)
    for b in (0, 7, 31, 63, max(range(64), key=lambda i: ctx[i])):
        kb, vb, tb = _gather_request(kc, vc, table, b, ctx[b], page)
        ref, ref_lse = attention_reference(q[b], kb, vb, torch.tensor([0, 1], dtype=torch.int32),
                                           used_k=torch.tensor([ctx[b]]), block_table=tb)
        assert_north_star(out[b], lse[b], ref, ref_lse, torch.bfloat16)


def test_config3_store_kvcache_bytes(device):
    """store_kvcache of config 3's first requests: every slot holds its token's
    bits (scatter then gather is the identity), as the oracle scatter says."""
    g = torch.Generator().manual_seed(123 + 3)
    ctx = torch.randint(512, 32769, (64,), generator=g).tolist()[:6]
    hkv, d, page = 8, 128, 16
    kc, vc, table, slots = bench.paged_cache(ctx, page, hkv, d, torch.bfloat16, device, 123 + 3)
    gdev = torch.Generator(device=device).manual_seed(123 + 3)
    kx = torch.randn(sum(ctx), hkv, d, generator=gdev, device=device, dtype=torch.float32).to(torch.bfloat16)
    vx = torch.randn(sum(ctx), hkv, d, generator=gdev, device=device, dtype=torch.float32).to(torch.bfloat16)
    flat_k = kc.view(-1, hkv, d)[slots.long()].cpu()
    flat_v = vc.view(-1, hkv, d)[slots.long()].cpu()
    assert torch.equal(flat_k.view(torch.int16), kx.cpu().view(torch.int16))
    assert torch.equal(flat_v.view(torch.int16), vx.cpu().view(torch.int16))
    sub = slice(0, 2000)
    expect = ocache.store_kvcache(kx[sub].cpu(), torch.zeros(kc.shape, dtype=kc.dtype), slots[sub].cpu())
    written = expect.view(-1, hkv, d)[slots[sub].long().cpu()]
    assert torch.equal(written.view(torch.int16), flat_k[sub].view(torch.int16))


def test_config4_fp8_paged_decode_full_size(device):
    g = torch.Generator().manual_seed(123 + 4)
    ctx = torch.randint(1024, 8193, (128,), generator=g).tolist()
    hq, hkv, d, page = 16, 8, 256, 16
    scale = torch.empty(hkv).uniform_(0.01, 0.1, generator=g)
    kc, vc, table, slots = bench.paged_cache(ctx, page, hkv, d, torch.float8_e4m3fn, device, 123 + 4,
                                             scale=scale.to(device))
    q = torch.randn(128, hq, d, generator=g).to(torch.bfloat16).to(device)
    cuq = torch.arange(129, dtype=torch.int32, device=device)
    used = torch.tensor(ctx, dtype=torch.int32, device=device)
    desc = scale.to(device).expand(128, hkv)
    out, lse = vllm.flash_attn_varlen_func(q, kc, vc, 1, cuq, max(ctx), seqused_k=used, block_table=table,
                                           causal=True, softcap=50.0, window_size=(4095, 0), k_descale=desc,
                                           v_descale=desc, return_softmax_lse=True)
    for b in (0, 5, 64, 127):
        kb, vb, tb = _gather_request(kc, vc, table, b, ctx[b], page)
        ref, ref_lse = attention_reference(q[b:b + 1], kb, vb, torch.tensor([0, 1], dtype=torch.int32),
                                           used_k=torch.tensor([ctx[b]]), block_table=tb, softcap=50.0,
                                           window=(4095, 0), k_descale=desc[b:b + 1].cpu(),
                                           v_descale=desc[b:b + 1].cpu())
        assert_north_star(out[b:b + 1], lse[:, b:b + 1], ref, ref_lse, torch.bfloat16)
    # the FP8 cache bytes of the first request equal the C codec of x / scale
    gdev = torch.Generator(device=device).manual_seed(123 + 4)
    kx = torch.randn(sum(ctx), hkv, d, generator=gdev, device=device, dtype=torch.float32).to(torch.bfloat16)
    n0 = ctx[0]
    pos = torch.arange(n0)
    tb = table[0].cpu()
    got = kc.view(torch.uint8)[tb[pos // page].long().to(device), (pos % page).to(device)].cpu()
    from oracle import fp8 as ofp8
    want = ofp8.encode_scaled(kx[:n0].float().cpu().numpy(), scale.numpy())
    assert torch.equal(got, torch.from_numpy(want))


def test_config5_mixed_diffkv_full_size(device):
    g = torch.Generator().manual_seed(123 + 5)
    hq = hkv = 16
    dqk, dv, page = 192, 128, 16
    prefixes = torch.randint(0, 4097, (8,), generator=g).tolist()
    dec_ctx = torch.randint(256, 16385, (120,), generator=g).tolist()
    q_lens = [512] * 8 + [1] * 120
    k_lens = [p + 512 for p in prefixes] + dec_ctx
    kc, vc, table, _ = bench.paged_cache(k_lens, page, hkv, dqk, torch.bfloat16, device, 123 + 5, dv=dv)
    total_q = sum(q_lens)
    q = torch.randn(total_q, hq, dqk, generator=g).to(torch.bfloat16).to(device)
    sinks = torch.randn(hq, generator=g).to(device)
    cuq = cu_from_lengths(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    storage = torch.full((total_q + 4, hq, dv), 5.0, dtype=torch.bfloat16, device=device)
    out = storage[2:total_q + 2]
    res, lse = vllm.flash_attn_varlen_func(q, kc, vc, max(q_lens), cuq, max(k_lens), seqused_k=used,
                                           block_table=table, causal=True, s_aux=sinks, out=out,
                                           return_softmax_lse=True)
    assert res.data_ptr() == out.data_ptr()
    assert torch.all(storage[:2] == 5.0) and torch.all(storage[-2:] == 5.0)
    starts = [0]
    for n in q_lens:
        starts.append(starts[-1] + n)
    for b in (0, 3, 7, 8, 50, 127):
        kb, vb, tb = _gather_request(kc, vc, table, b, k_lens[b], page)
        qs = q[starts[b]:starts[b + 1]]
        rows = _sample_rows([q_lens[b]], per_request=16, seed=b)
        ref, ref_lse = attention_reference(qs, kb, vb, torch.tensor([0, q_lens[b]], dtype=torch.int32),
                                           used_k=torch.tensor([k_lens[b]]), block_table=tb, causal=True,
                                           sinks=sinks, rows=rows)
        assert_north_star(out[starts[b]:starts[b + 1]], lse[:, starts[b]:starts[b + 1]], ref, ref_lse,
                          torch.bfloat16, rows=rows)
