"""vLLM FLASH_ATTN / FLASH_ATTN_DIFFKV contract on gfx950 against the CPU oracle.

Request shapes and feature values are data from flash_attn_mps
tests/test_vllm.py (cited per case); the checks are this build's parity bar
(fp16 2e-3, bf16 1e-2, LSE 1e-4 max-abs), caller-owned outputs with
untouched sentinels, and bit-exact batch invariance.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd.vllm import flash_attn_varlen_func, merge_attn_states, mm_prefix_mask, rswa_mask
from harness import assert_parity, offsets, oracle_attention, seeded

pytestmark = pytest.mark.gpu


def _requests(device, q_lens, k_lens, dqk, dv, seed, dtype=torch.float16):
    """Packed q [sum q_lens, 4, dqk], k/v [sum k_lens, 2, d] and their offsets."""
    q = seeded((sum(q_lens), 4, dqk), seed, dtype, device)
    k = seeded((sum(k_lens), 2, dqk), seed + 1, dtype, device)
    v = seeded((sum(k_lens), 2, dv), seed + 2, dtype, device)
    lengths = dict(cu_seqlens_q=offsets(q_lens, device), cu_seqlens_k=offsets(k_lens, device),
                   max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens))
    return q, k, v, lengths


@pytest.mark.parametrize("causality", ["causal", "bidirectional", "per-request"])
def test_all_score_features_into_a_caller_buffer(device, causality):
    """Window (15, 15), softcap 2, ALiBi slopes, sinks and fa_version 4, written
    into a strided view of a sentinel-filled buffer (test_vllm.py:18-37:
    q lengths 1/4/17, k lengths 65/100/17, d 64 / dv 32)."""
    q, k, v, lengths = _requests(device, (1, 4, 17), (65, 100, 17), 64, 32, seed=300)
    per_request = torch.tensor([True, False, True], device=device)
    slopes = torch.tensor([0.1, 0.2, 0.3, 0.4], device=device)
    sinks = torch.tensor([-1.0, 0.0, 1.0, 2.0], device=device)
    buffer = torch.full((q.shape[0] + 5, 4, 32), 123.0, device=device, dtype=q.dtype)
    out = buffer[: q.shape[0]]
    causal = {"causal": True, "bidirectional": False, "per-request": True}[causality]
    dynamic = per_request if causality == "per-request" else None
    got, lse = flash_attn_varlen_func(q, k, v, **lengths, causal=causal, dynamic_causal=dynamic,
                                      window_size=[15, 15], softcap=2.0, alibi_slopes=slopes, s_aux=sinks,
                                      out=out, return_softmax_lse=True, fa_version=4)
    assert got.data_ptr() == out.data_ptr()
    assert (buffer[q.shape[0]:] == 123).all()
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], lengths["cu_seqlens_k"],
                                    causal=per_request if dynamic is not None else causal, window=(15, 15),
                                    softcap=2.0, alibi=slopes, sinks=sinks)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("mask_name", ["prefix", "prefix+window", "prefix clamped to window", "rolling window"])
def test_mask_descriptors_over_a_poisoned_paged_cache(device, mask_name):
    """96 queries over 257 keys in 64-token pages [5, 1, 7, 3, 0]; every slot
    past the sequence is NaN; rows 31-60 also see keys 192-221
    (test_vllm.py:40-66)."""
    q, k_packed, v_packed, lengths = _requests(device, (96,), (257,), 64, 32, seed=310)
    table = torch.tensor([[5, 1, 7, 3, 0]], device=device, dtype=torch.int32)
    k = torch.full((8, 64, 2, 64), float("nan"), device=device, dtype=q.dtype)
    v = torch.full((8, 64, 2, 32), float("nan"), device=device, dtype=q.dtype)
    pos = torch.arange(257, device=device)
    pages = table[0, pos // 64].long()
    k[pages, pos % 64], v[pages, pos % 64] = k_packed, v_packed
    used = torch.tensor([257], device=device, dtype=torch.int32)
    ranges = torch.full((96, 2), -1, device=device, dtype=torch.int32)
    ranges[31:61] = torch.tensor([192, 221], device=device, dtype=torch.int32)
    if mask_name == "rolling window":
        mask = rswa_mask()
        aux = [torch.tensor([64], device=device, dtype=torch.int32),
               torch.tensor([16], device=device, dtype=torch.int32)]
    else:
        mask = mm_prefix_mask(None if mask_name == "prefix" else 16, mask_name == "prefix clamped to window")
        aux = [ranges, lengths["cu_seqlens_q"]]
    got, lse = flash_attn_varlen_func(q, k, v, 96, lengths["cu_seqlens_q"], 257, seqused_k=used,
                                      block_table=table, mask_mod=mask, aux_tensors=aux,
                                      return_softmax_lse=True, fa_version=4)
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], used_k=used, block_table=table,
                                    mask=mask, aux=aux)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("mask_name", ["prefix", "prefix+window", "prefix clamped to window", "rolling window"])
def test_mask_descriptors_run_on_the_mfma_prefill(device, mask_name, monkeypatch):
    """The same mask calls at dq = dv = 64 (the dims the MFMA prefill takes
    mask kinds at) go to fa_prefill_fwd, not to the generic kernel, and meet
    the parity bar."""
    q, k_packed, v_packed, lengths = _requests(device, (96,), (257,), 64, 64, seed=320)
    table = torch.tensor([[5, 1, 7, 3, 0]], device=device, dtype=torch.int32)
    k = torch.full((8, 64, 2, 64), float("nan"), device=device, dtype=q.dtype)
    v = torch.full((8, 64, 2, 64), float("nan"), device=device, dtype=q.dtype)
    pos = torch.arange(257, device=device)
    pages = table[0, pos // 64].long()
    k[pages, pos % 64], v[pages, pos % 64] = k_packed, v_packed
    used = torch.tensor([257], device=device, dtype=torch.int32)
    ranges = torch.full((96, 2), -1, device=device, dtype=torch.int32)
    ranges[31:61] = torch.tensor([192, 221], device=device, dtype=torch.int32)
    if mask_name == "rolling window":
        mask = rswa_mask()
        aux = [torch.tensor([64], device=device, dtype=torch.int32),
               torch.tensor([16], device=device, dtype=torch.int32)]
    else:
        mask = mm_prefix_mask(None if mask_name == "prefix" else 16, mask_name == "prefix clamped to window")
        aux = [ranges, lengths["cu_seqlens_q"]]
    calls = []
    real_call = _lib.call
    monkeypatch.setattr(_lib, "call", lambda name, *a, **kw: (calls.append(name), real_call(name, *a, **kw))[1])
    got, lse = flash_attn_varlen_func(q, k, v, 96, lengths["cu_seqlens_q"], 257, seqused_k=used,
                                      block_table=table, mask_mod=mask, aux_tensors=aux,
                                      return_softmax_lse=True, fa_version=4)
    assert "fa_prefill_fwd" in calls and "fa_attn_fwd" not in calls, calls
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], used_k=used, block_table=table,
                                    mask=mask, aux=aux)
    assert_parity(got, lse, ref, ref_lse)


def test_fp8_queries_keys_values_with_broadcast_descales(device):
    """E4M3 q/k/v with [B, Hkv] descales given as stride-0 expansions; the
    output defaults to fp16 (test_vllm.py:69-82: lengths 3/7 and 19/23)."""
    q, k, v, lengths = _requests(device, (3, 7), (19, 23), 32, 64, seed=320)
    q, k, v = (t.cpu().to(torch.float8_e4m3fn).to(device) for t in (q, k, v))
    qd = torch.tensor([[0.8, 1.2]], device=device).expand(2, 2)
    kd = torch.tensor([[0.3], [0.7]], device=device).expand(2, 2)
    vd = torch.tensor([[0.9, 1.1]], device=device).expand(2, 2)
    got, lse = flash_attn_varlen_func(q, k, v, **lengths, q_descale=qd, k_descale=kd, v_descale=vd,
                                      causal=True, return_softmax_lse=True, fa_version=3)
    assert got.dtype == torch.float16
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], lengths["cu_seqlens_k"], causal=True,
                                    q_descale=qd, k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


def _slice_call(q, k, v, cu_q, max_q, lo, hi, **kw):
    cu_k = torch.tensor([0, hi - lo], device=q.device, dtype=torch.int32)
    return flash_attn_varlen_func(q, k[lo:hi], v[lo:hi], max_q, cu_q, hi - lo, cu_seqlens_k=cu_k,
                                  return_softmax_lse=True, **kw)


def test_cascade_merge_of_key_ranges_equals_the_full_call(device):
    """Keys 0-63, an empty range and keys 64-128, attended separately and
    merged pairwise in place (test_vllm.py:85-101)."""
    q, k, v, lengths = _requests(device, (4,), (129,), 32, 64, seed=330)
    full, full_lse = flash_attn_varlen_func(q, k, v, **lengths, return_softmax_lse=True)
    parts = [_slice_call(q, k, v, lengths["cu_seqlens_q"], 4, lo, hi) for lo, hi in ((0, 64), (64, 64), (64, 129))]
    out, out_lse = torch.empty_like(full), torch.empty_like(full_lse)
    merge_attn_states(out, *parts[0], *parts[1], output_lse=out_lse)
    merge_attn_states(out, out.clone(), out_lse.clone(), *parts[2], output_lse=out_lse)
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], lengths["cu_seqlens_k"])
    assert_parity(out, out_lse, ref, ref_lse, what="merged")
    assert_parity(full, full_lse, ref, ref_lse, what="full")


@pytest.mark.parametrize("splits", [1, 2, 4, 7])
def test_explicit_split_counts(device, splits):
    """A decode row and a 4-row chunk over 1025 / 513 keys (test_vllm.py:104-110)."""
    q, k, v, lengths = _requests(device, (1, 4), (1025, 513), 64, 64, seed=340)
    got, lse = flash_attn_varlen_func(q, k, v, **lengths, causal=True, num_splits=splits, return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], lengths["cu_seqlens_k"], causal=True)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("page", [16, 32, 64, 128, 256])
def test_fp8_paged_cache_with_bf16_queries(device, page):
    """K and V are the two halves of one E4M3 [pages, heads, P, 128] buffer,
    read with bf16 queries and broadcast descales (test_vllm.py:113-131)."""
    raw = seeded((7, 2, page, 128), 350 + page, torch.float8_e4m3fn, device)
    k, v = raw.transpose(1, 2).split(64, -1)
    q = seeded((5, 4, 64), 351, torch.bfloat16, device)
    cu_q = torch.tensor([0, 1, 5], device=device, dtype=torch.int32)
    used = torch.tensor([page + 1, 2 * page - 1], device=device, dtype=torch.int32)
    table = torch.tensor([[4, 1], [5, 2]], device=device, dtype=torch.int32)
    kd = torch.tensor([[0.7, 1.2]], device=device).expand(2, 2)
    vd = torch.tensor([[0.9], [1.1]], device=device).expand(2, 2)
    got, lse = flash_attn_varlen_func(q, k, v, 4, cu_q, 2 * page, seqused_k=used, block_table=table, causal=True,
                                      k_descale=kd, v_descale=vd, return_softmax_lse=True, fa_version=4)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, used_k=used, block_table=table, causal=True,
                                    k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


def test_sink_counts_once_across_splits_and_merges(device):
    """One query over 513 keys with per-head sinks: split four ways, and as a
    prefix call (with the sink) merged with a suffix call (without)
    (test_vllm.py:134-155)."""
    q, k, v, lengths = _requests(device, (1,), (513,), 32, 32, seed=360)
    sinks = torch.tensor([1.0, 2.0, 3.0, 4.0], device=device)
    ref, ref_lse = oracle_attention(q, k, v, lengths["cu_seqlens_q"], lengths["cu_seqlens_k"], sinks=sinks)
    split, split_lse = flash_attn_varlen_func(q, k, v, **lengths, s_aux=sinks, num_splits=4, return_softmax_lse=True)
    assert_parity(split, split_lse, ref, ref_lse, what="split")
    prefix = _slice_call(q, k, v, lengths["cu_seqlens_q"], 1, 0, 256, s_aux=sinks)
    suffix = _slice_call(q, k, v, lengths["cu_seqlens_q"], 1, 256, 513)
    out, out_lse = torch.empty_like(split), torch.empty_like(split_lse)
    merge_attn_states(out, *prefix, *suffix, output_lse=out_lse)
    assert_parity(out, out_lse, ref, ref_lse, what="merged")


def test_one_split_gives_batch_invariant_rows(device):
    """num_splits=1: a request's rows do not depend on what else is in the
    batch (test_vllm.py:158-167: a decode row batched with a 17-row chunk)."""
    q, k, v, lengths = _requests(device, (1, 17), (513, 529), 64, 64, seed=370)
    batched = flash_attn_varlen_func(q, k, v, **lengths, causal=True, num_splits=1)
    alone = _slice_call(q[:1], k, v, lengths["cu_seqlens_q"][:2], 1, 0, 513, causal=True, num_splits=1)[0]
    assert torch.equal(alone, batched[:1])
