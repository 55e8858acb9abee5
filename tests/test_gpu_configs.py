"""The five benchmark configurations at full size, every output row against
the CPU oracle at the parity bar (bf16 1e-2, fp16 2e-3, fp32 1e-4, LSE 1e-4).

Inputs come from bench.py's own builders, so these are the exact tensors the
benchmark times.  Full-size sweeps run the oracle in float32 and in chunks of
rows (rows are independent, so chunking is exact; float32 attention over at
most 32K keys is within ~1e-6 of float64, far inside the bar).  Decode
requests are checked one by one on their gathered pages, every request.
Cache bytes written by store_kvcache are checked exactly.
"""
import pytest
import torch

import bench
from flash_attn_mps_amd import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache, vllm
from harness import assert_parity, offsets, oracle_attention
from oracle import cache as ocache
from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu


def _request_pages(k_cache, v_cache, table, b, length, page):
    """Request b's pages copied to the CPU, with a table addressing them in order."""
    n = -(-length // page)
    pages = table[b, :n].long()
    return k_cache[pages].cpu(), v_cache[pages].cpu(), torch.arange(n, dtype=torch.int32).reshape(1, n)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_config1_dense_causal_gqa(device, dtype):
    """Batch 2 x 128 tokens, 16/8 heads, d 128, N(0,1) from seed 124, every row (fp64 oracle)."""
    g = torch.Generator().manual_seed(123 + 1)
    q, k, v = (torch.randn(2, 128, h, 128, generator=g).to(dtype) for h in (16, 8, 8))
    out, lse = flash_attn_func(q.to(device), k.to(device), v.to(device), softmax_scale=128 ** -0.5, causal=True,
                               return_softmax_lse=True)
    assert out.shape == (2, 128, 16, 128) and lse.shape == (2, 16, 128)
    cu = offsets([128, 128])
    ref, ref_lse = oracle_attention(q.flatten(0, 1), k.flatten(0, 1), v.flatten(0, 1), cu, cu, causal=True)
    assert_parity(out.flatten(0, 1), lse.transpose(0, 1).flatten(1), ref, ref_lse, dtype)


def test_config2_every_row(device):
    """All 36.5K query rows x 16 heads of the headline prefill."""
    c = bench.config2_inputs(device)
    q, k, v, cu, lengths = c["q"], c["k"], c["v"], c["cu"], c["lengths"]
    out, lse = flash_attn_varlen_func(q, k, v, cu, cu, max(lengths), max(lengths), causal=True,
                                      return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, k, v, cu, cu, causal=True, dtype=torch.float32, chunk=2048)
    errors = assert_parity(out, lse, ref, ref_lse, torch.bfloat16, what="config 2")
    print(f"config 2: max |out - oracle| {errors[0]:.3e}, max |lse - oracle| {errors[1]:.3e}")


def test_config2_lengths_with_unit_normal_values(device):
    """Config 2's lengths and Q/K with V ~ N(0, 1) (config 2 draws 0.5 N(0, 1);
    doubling is exact in bf16): the MFMA kernel rounds the softmax weights to
    bf16 before P.V, which bounds a row's error by about 2^-8 max|v|; every
    row still meets the 1e-2 bar."""
    c = bench.config2_inputs(device)
    q, k, v, cu, lengths = c["q"], c["k"], c["v"] * 2, c["cu"], c["lengths"]
    out, lse = flash_attn_varlen_func(q, k, v, cu, cu, max(lengths), max(lengths), causal=True,
                                      return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, k, v, cu, cu, causal=True, dtype=torch.float32, chunk=2048)
    errors = assert_parity(out, lse, ref, ref_lse, torch.bfloat16, what="config 2, V ~ N(0, 1)")
    print(f"config 2 with N(0,1) V: max |out - oracle| {errors[0]:.3e}, max |lse - oracle| {errors[1]:.3e}")


def test_config3_every_request(device):
    """All 64 single-query requests over 512-32768 keys in permuted 16-token pages."""
    c = bench.config3_inputs(device)
    out, lse = flash_attn_with_kvcache(c["q"], c["k_cache"], c["v_cache"], cache_seqlens=c["lengths"],
                                       block_table=c["table"], causal=True, return_softmax_lse=True)
    worst = [0.0, 0.0]
    for b, length in enumerate(c["ctx"]):
        kb, vb, tb = _request_pages(c["k_cache"], c["v_cache"], c["table"], b, length, c["page"])
        ref, ref_lse = oracle_attention(c["q"][b], kb, vb, offsets([1]), used_k=torch.tensor([length]), block_table=tb)
        errs = assert_parity(out[b], lse[b], ref, ref_lse, torch.bfloat16, what=f"config 3 request {b}")
        worst = [max(w, e) for w, e in zip(worst, errs)]
    print(f"config 3: max |out - oracle| {worst[0]:.3e}, max |lse - oracle| {worst[1]:.3e}")


def test_config3_cache_bytes(device):
    """store_kvcache put every one of config 3's 1.07M tokens at its slot: the
    cache gathered through the slot map equals the source rows, bit for bit,
    and the oracle scatter of a sample agrees."""
    c = bench.config3_inputs(device)
    hkv, d = c["kv_heads"], c["dim"]
    g = torch.Generator(device=device).manual_seed(123 + 3)
    tokens = sum(c["ctx"])
    kx = torch.randn(tokens, hkv, d, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    vx = torch.randn(tokens, hkv, d, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    slots = c["slots"].long()
    assert torch.equal(c["k_cache"].view(-1, hkv, d)[slots].view(torch.int16), kx.view(torch.int16))
    assert torch.equal(c["v_cache"].view(-1, hkv, d)[slots].view(torch.int16), vx.view(torch.int16))
    sample = slice(0, 2000)
    expect = ocache.store_kvcache(kx[sample].cpu(), torch.zeros(c["k_cache"].shape, dtype=torch.bfloat16),
                                  c["slots"][sample].cpu())
    written = expect.view(-1, hkv, d)[slots[sample].cpu()]
    assert torch.equal(written.view(torch.int16), kx[sample].cpu().view(torch.int16))


def test_config4_every_request(device):
    """All 128 FP8 decode requests (softcap 50, window 4095, descales), and
    the E4M3 bytes of every cached key equal the C codec of x / scale."""
    c = bench.config4_inputs(device)
    out, lse = vllm.flash_attn_varlen_func(c["q"], c["k_cache"], c["v_cache"], 1, c["cu_q"], max(c["ctx"]),
                                           seqused_k=c["lengths"], block_table=c["table"], causal=True,
                                           softcap=c["softcap"], window_size=c["window"], k_descale=c["descale"],
                                           v_descale=c["descale"], return_softmax_lse=True)
    worst = [0.0, 0.0]
    for b, length in enumerate(c["ctx"]):
        kb, vb, tb = _request_pages(c["k_cache"], c["v_cache"], c["table"], b, length, c["page"])
        ref, ref_lse = oracle_attention(c["q"][b:b + 1], kb, vb, offsets([1]), used_k=torch.tensor([length]),
                                        block_table=tb, softcap=c["softcap"], window=c["window"],
                                        k_descale=c["descale"][b:b + 1].cpu(), v_descale=c["descale"][b:b + 1].cpu())
        errs = assert_parity(out[b:b + 1], lse[:, b:b + 1], ref, ref_lse, torch.bfloat16,
                             what=f"config 4 request {b}")
        worst = [max(w, e) for w, e in zip(worst, errs)]
    print(f"config 4: max |out - oracle| {worst[0]:.3e}, max |lse - oracle| {worst[1]:.3e}")
    hkv, d = c["kv_heads"], c["dim"]
    g = torch.Generator(device=device).manual_seed(123 + 4)
    kx = torch.randn(sum(c["ctx"]), hkv, d, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    stored = c["k_cache"].view(torch.uint8).view(-1, hkv, d)[c["slots"].long()].cpu()
    expected = ofp8.encode_scaled(kx.float().cpu().numpy(), c["scale"].numpy())
    assert torch.equal(stored, torch.from_numpy(expected))


def test_config5_every_row(device):
    """All 4096 chunk rows and 120 decode rows of the mixed DIFFKV call, with
    sinks, into a caller buffer whose margins must stay untouched."""
    c = bench.config5_inputs(device)
    q_lens, k_lens, page = c["q_lens"], c["k_lens"], c["page"]
    total = sum(q_lens)
    buffer = torch.full((total + 4, c["heads"], c["dim_v"]), 5.0, dtype=torch.bfloat16, device=device)
    out = buffer[2:total + 2]
    got, lse = vllm.flash_attn_varlen_func(c["q"], c["k_cache"], c["v_cache"], max(q_lens), c["cu_q"], max(k_lens),
                                           seqused_k=c["used"], block_table=c["table"], causal=True,
                                           s_aux=c["sinks"], out=out, return_softmax_lse=True)
    assert got.data_ptr() == out.data_ptr()
    assert (buffer[:2] == 5.0).all() and (buffer[-2:] == 5.0).all()
    starts = [0]
    for n in q_lens:
        starts.append(starts[-1] + n)
    worst = [0.0, 0.0]
    for b, (lq, lk) in enumerate(zip(q_lens, k_lens)):
        kb, vb, tb = _request_pages(c["k_cache"], c["v_cache"], c["table"], b, lk, page)
        rows = slice(starts[b], starts[b + 1])
        ref, ref_lse = oracle_attention(c["q"][rows], kb, vb, offsets([lq]), used_k=torch.tensor([lk]),
                                        block_table=tb, causal=True, sinks=c["sinks"], dtype=torch.float32)
        errs = assert_parity(out[rows], lse[:, rows], ref, ref_lse, torch.bfloat16, what=f"config 5 request {b}")
        worst = [max(w, e) for w, e in zip(worst, errs)]
    print(f"config 5: max |out - oracle| {worst[0]:.3e}, max |lse - oracle| {worst[1]:.3e}")
