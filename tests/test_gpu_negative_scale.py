"""A negative softmax scale on every route (the score is scale * q.k for any
sign): the row max must be that of the scaled scores, and a masked key must
keep zero weight (-inf times a negative scale is +inf).  The VALU decode,
the matrix-core decode (one row and several rows per request), the generic
kernel (fp32) and a mixed batch, each against the oracle at the parity bar.
"""
import pytest
import torch

from flash_attn_mps_amd._decode import uses_gqa_kernel
from harness import assert_parity, attention, decode_attention, offsets, oracle_attention, problem

pytestmark = pytest.mark.gpu

SCALE = -128 ** -0.5


def _paged(lengths, kv_heads, d, dtype, seed, spread=1.0, page=16):
    g = torch.Generator().manual_seed(seed)
    cols = max(-(-n // page) for n in lengths) + 1
    table = torch.randperm(len(lengths) * cols, generator=g).int().reshape(len(lengths), cols)
    kc = (torch.randn(len(lengths) * cols, page, kv_heads, d, generator=g) * spread).to(dtype)
    vc = (torch.randn(len(lengths) * cols, page, kv_heads, d, generator=g) * 0.25).to(dtype)
    return kc, vc, table, cols * page


@pytest.mark.parametrize("heads,kv_heads", [(16, 8), (32, 4), (24, 8)])
@pytest.mark.parametrize("window", [(-1, -1), (100, 0)])
def test_decode_negative_scale(device, heads, kv_heads, window):
    lengths = [1, 40, 777, 2049, 300]
    kc, vc, table, max_k = _paged(lengths, kv_heads, 128, torch.bfloat16, 900 + heads, spread=2.0)
    g = torch.Generator().manual_seed(901)
    q = (torch.randn(len(lengths), heads, 128, generator=g) * 2.0).to(torch.bfloat16)
    cu_q, used = offsets([1] * len(lengths)), torch.tensor(lengths, dtype=torch.int32)
    kw = dict(cu_seqlens_q=cu_q.to(device), seqused_k=used.to(device), block_table=table.to(device),
              softmax_scale=SCALE, window_size=window)
    p = problem(q.to(device), kc.to(device), vc.to(device), max_seqlen_q=1, max_seqlen_k=max_k, **kw)
    assert uses_gqa_kernel(p) == (heads // kv_heads >= 3)
    out, lse = decode_attention(q.to(device), kc.to(device), vc.to(device), max_seqlen_k=max_k, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, scale=SCALE, window=window)
    assert_parity(out, lse, ref, ref_lse)


@pytest.mark.parametrize("causal", [True, False])
def test_multi_row_decode_negative_scale(device, causal):
    q_lens, lengths = [4, 1, 3, 4], [50, 900, 3, 2000]
    kc, vc, table, max_k = _paged(lengths, 8, 128, torch.bfloat16, 910, spread=2.0)
    g = torch.Generator().manual_seed(911)
    q = (torch.randn(sum(q_lens), 32, 128, generator=g) * 2.0).to(torch.bfloat16)
    cu_q, used = offsets(q_lens), torch.tensor(lengths, dtype=torch.int32)
    kw = dict(cu_seqlens_q=cu_q.to(device), seqused_k=used.to(device), block_table=table.to(device),
              softmax_scale=SCALE, causal=causal, max_seqlen_q=max(q_lens), max_seqlen_k=max_k)
    assert uses_gqa_kernel(problem(q.to(device), kc.to(device), vc.to(device), **kw))
    out, lse = attention(q.to(device), kc.to(device), vc.to(device), **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, scale=SCALE, causal=causal)
    assert_parity(out, lse, ref, ref_lse)


def test_generic_kernel_negative_scale(device):
    """fp32 inputs take the generic kernel."""
    q_lens, k_lens = [3, 70, 200], [10, 70, 260]
    g = torch.Generator().manual_seed(920)
    q = torch.randn(sum(q_lens), 4, 64, generator=g) * 2.0
    k = torch.randn(sum(k_lens), 2, 64, generator=g) * 2.0
    v = torch.randn(sum(k_lens), 2, 64, generator=g) * 0.5
    cuq, cuk = offsets(q_lens), offsets(k_lens)
    kw = dict(cu_seqlens_q=cuq.to(device), cu_seqlens_k=cuk.to(device), max_seqlen_q=max(q_lens),
              max_seqlen_k=max(k_lens), causal=True, softmax_scale=SCALE)
    out, lse = attention(q.to(device), k.to(device), v.to(device), **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, scale=SCALE)
    assert_parity(out, lse, ref, ref_lse)


def test_mixed_batch_negative_scale(device):
    """Chunked-prefill requests on the MFMA prefill and single-query requests
    on the decode kernel in one call."""
    q_lens, lengths = [1, 300, 1, 1, 129], [700, 500, 1, 2000, 129]
    kc, vc, table, max_k = _paged(lengths, 8, 128, torch.bfloat16, 930, spread=2.0)
    g = torch.Generator().manual_seed(931)
    q = (torch.randn(sum(q_lens), 16, 128, generator=g) * 2.0).to(torch.bfloat16)
    cu_q, used = offsets(q_lens), torch.tensor(lengths, dtype=torch.int32)
    kw = dict(cu_seqlens_q=cu_q.to(device), seqused_k=used.to(device), block_table=table.to(device),
              softmax_scale=SCALE, causal=True, max_seqlen_q=max(q_lens), max_seqlen_k=max_k)
    out, lse = attention(q.to(device), kc.to(device), vc.to(device), **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, scale=SCALE, causal=True)
    assert_parity(out, lse, ref, ref_lse)
