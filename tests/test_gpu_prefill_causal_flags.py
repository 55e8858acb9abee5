"""Per-request causality (vLLM's dynamic_causal) on the MFMA prefill kernel.

A bool [B] tensor marks which requests are causal
(flash_attn_mps/_attention.py:88-238 takes `causal` as a tensor; the mask is
kernels/attention.metal:29-45).  The kernel runs such calls in its window
variant with a right window of 0 for causal requests.  Covered: both grid
modes (compact work list with Hkv a multiple of 8, per-pair grid otherwise),
more than 64 requests, q_len != k_len, left windows, paged K/V, single-query
requests in the batch, and the route.  Tolerances: max-abs <= 1e-2 bf16,
<= 2e-3 fp16, LSE <= 1e-4.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd.vllm import flash_attn_varlen_func
from harness import assert_parity, attention, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu


def _inputs(device, dtype, hq, hkv, d, q_lens, k_lens, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(dtype).to(device)
    k = (torch.randn(sum(k_lens), hkv, d, generator=g) * 0.5).to(dtype).to(device)
    v = torch.randn(sum(k_lens), hkv, d, generator=g).to(dtype).to(device)
    flags = torch.rand(len(q_lens), generator=g) < 0.5
    flags[0], flags[-1] = True, False
    return q, k, v, offsets(q_lens, device), offsets(k_lens, device), flags.to(device)


def _routes_to_mfma(q, k, v, **kw):
    out = torch.empty(q.shape[0], q.shape[1], v.shape[-1], dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[1], q.shape[0], device=q.device)
    full = dict(cu_seqlens_q=None, cu_seqlens_k=None, seqused_k=None, max_seqlen_q=1, max_seqlen_k=1,
                block_table=None, softmax_scale=None, causal=False, window_size=(-1, -1), alibi_slopes=None,
                softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None, mask_mod=None,
                aux_tensors=None, leftpad_k=None)
    full.update(kw)
    keep = []
    return _lib.supported("fa_prefill_supported", kernel_args(q, k, v, out, lse, keep=keep, **full))


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 2)])
@pytest.mark.parametrize("window", [(-1, -1), (100, -1), (64, 32)])
def test_causal_flags_packed(device, hq, hkv, window):
    q_lens, k_lens = [300, 1, 129, 64, 513, 40], [300, 77, 200, 64, 700, 10]
    q, k, v, cuq, cuk, flags = _inputs(device, torch.bfloat16, hq, hkv, 128, q_lens, k_lens, seed=hq + window[0])
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=flags, window_size=window)
    assert _routes_to_mfma(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=flags, window=window)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_causal_flags_many_requests(device):
    """100 requests: the compact work list's four-per-lane ranking."""
    g = torch.Generator().manual_seed(7)
    q_lens = torch.randint(1, 200, (100,), generator=g).tolist()
    k_lens = [n + int(torch.randint(0, 50, (1,), generator=g)) for n in q_lens]
    q, k, v, cuq, cuk, flags = _inputs(device, torch.float16, 16, 8, 64, q_lens, k_lens, seed=8)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens),
                         max_seqlen_k=max(k_lens), causal=flags)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=flags)
    assert_parity(out, lse, ref, ref_lse, torch.float16)


@pytest.mark.parametrize("page", [16, 64])
def test_dynamic_causal_vllm_paged(device, page):
    """vllm.flash_attn_varlen_func(dynamic_causal=...) over a paged cache with NaN-poisoned slots."""
    g = torch.Generator().manual_seed(page)
    q_lens, k_lens = [200, 1, 96, 33], [400, 130, 96, 300]
    hq, hkv, d = 8, 8, 128
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens) + 2
    table = torch.randperm(pool, generator=g)[:cols * len(k_lens)].int().reshape(len(k_lens), cols)
    kc = torch.full((pool, page, hkv, d), float("nan"))
    vc = torch.full((pool, page, hkv, d), float("nan"))
    for b, n in enumerate(k_lens):
        for pos in range(n):
            kc[table[b, pos // page], pos % page] = torch.randn(hkv, d, generator=g) * 0.5
            vc[table[b, pos // page], pos % page] = torch.randn(hkv, d, generator=g)
    kc, vc = kc.to(torch.bfloat16).to(device), vc.to(torch.bfloat16).to(device)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    table = table.to(device)
    flags = torch.tensor([True, False, False, True], device=device)
    out, lse = flash_attn_varlen_func(q, kc, vc, max(q_lens), cuq, cols * page, seqused_k=used,
                                      block_table=table, causal=True, dynamic_causal=flags,
                                      return_softmax_lse=True, fa_version=4)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=flags)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
