"""vLLM mask kinds and left padding on the MFMA prefill kernel vs the CPU oracle.

Mask kind 1 is vllm.mm_prefix_mask (a causal / windowed part plus a per-row
modality key range that may lie past the diagonal), kind 2 is vllm.rswa_mask
(a prefix of global keys plus a per-row sliding window; the kernel runs the
prefix and the windows as two key passes when whole tiles lie between them).
Semantics: flash_attn_mps/kernels/attention.metal:29-45 (the oracle restates
them); mask descriptors and aux tensors as in flash_attn_mps/vllm.py:11-23 and
tests/test_vllm.py:40-66.  Left padding (flash_attn_with_kvcache's
cache_leftpad over a dense cache, interface.py:295-296) shifts a request's
storage positions.  Every case asserts that fa_prefill_fwd takes the call,
then holds outputs and LSE to this build's bar (bf16 1e-2, fp16 2e-3 max-abs,
LSE 1e-4 on every row; -inf LSE where no key is visible).
"""
import pytest
import torch

from flash_attn_mps_amd import _lib, flash_attn_with_kvcache
from flash_attn_mps_amd.vllm import mm_prefix_mask, rswa_mask
from harness import assert_parity, attention, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu

VALUE_SCALE = 0.5   # values as in config 2 (the MFMA P.V rounds P to 16 bits)
DIMS = [(64, 64), (128, 128), (192, 128), (256, 256)]


def _inputs(device, dtype, q_lens, k_lens, hq, hkv, dqk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(sum(q_lens), hq, dqk, generator=g) * 0.5).to(dtype).to(device)
    k = (torch.randn(sum(k_lens), hkv, dqk, generator=g) * 0.5).to(dtype).to(device)
    v = (torch.randn(sum(k_lens), hkv, dv, generator=g) * VALUE_SCALE).to(dtype).to(device)
    return q, k, v


def _paged(k, v, k_lens, page, device, seed):
    """Copy packed K/V into a shuffled pool of pages (unused slots NaN)."""
    g = torch.Generator().manual_seed(seed)
    n_pages = [-(-n // page) for n in k_lens]
    total = sum(n_pages) + 3
    perm = torch.randperm(total, generator=g)[: sum(n_pages)]
    table = torch.zeros(len(k_lens), max(n_pages), dtype=torch.int32)
    kc = torch.full((total, page) + tuple(k.shape[1:]), float("nan"), dtype=k.dtype, device=device)
    vc = torch.full((total, page) + tuple(v.shape[1:]), float("nan"), dtype=v.dtype, device=device)
    at, used = 0, 0
    for b, n in enumerate(k_lens):
        rows = perm[used: used + n_pages[b]]
        table[b, : n_pages[b]] = rows
        pos = torch.arange(n)
        kc[rows[pos // page].to(device), (pos % page).to(device)] = k[at: at + n]
        vc[rows[pos // page].to(device), (pos % page).to(device)] = v[at: at + n]
        at, used = at + n, used + n_pages[b]
    return kc, vc, table.to(device)


def _image_ranges(q_lens, k_lens, spans, device):
    """Kind 1 aux: [T, 2] absolute key ranges; rows whose absolute position
    lies in their request's image span [s0, s1) see the whole span (also the
    keys after them), others get -1."""
    rows = []
    for ql, kl, (s0, s1) in zip(q_lens, k_lens, spans):
        for i in range(ql):
            qa = i + kl - ql
            rows.append([s0, s1 - 1] if s0 <= qa < s1 else [-1, -1])
    return torch.tensor(rows, dtype=torch.int32, device=device)


def _check(device, q, k, v, dtype, what, **kw):
    out = torch.empty(q.shape[0], q.shape[1], v.shape[-1], dtype=q.dtype, device=device)
    lse = torch.empty(q.shape[1], q.shape[0], device=device)
    keep = []
    args = kernel_args(q, k, v, out, lse, keep=keep, **kw)
    assert _lib.supported("fa_prefill_supported", args), f"{what}: not on the MFMA prefill"
    got, got_lse = attention(q, k, v, **kw)
    oracle_kw = dict(cu_k=kw.get("cu_seqlens_k"), used_k=kw.get("seqused_k"), block_table=kw.get("block_table"),
                     mask=kw.get("mask_mod"), aux=kw.get("aux_tensors"), leftpad=kw.get("leftpad_k"),
                     softcap=kw.get("softcap", 0.0), k_descale=kw.get("k_descale"), v_descale=kw.get("v_descale"))
    ref, ref_lse = oracle_attention(q, k, v, kw["cu_seqlens_q"], **oracle_kw)
    assert_parity(got, got_lse, ref, ref_lse, dtype, what=what)


_NONE = dict(seqused_k=None, block_table=None, softmax_scale=None, causal=False, window_size=(-1, -1),
             alibi_slopes=None, softcap=0.0, s_aux=None, q_descale=None, k_descale=None, v_descale=None,
             leftpad_k=None)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dqk,dv", DIMS)
@pytest.mark.parametrize("window,clamp", [(None, False), (48, False), (48, True)])
def test_mm_prefix_mask(device, dtype, dqk, dv, window, clamp):
    """Chunked prefill rows over image spans: rows inside a span also see the
    span's later keys (past the diagonal); GQA 8/2 (two heads a workgroup)."""
    q_lens, k_lens = [200, 96, 37], [520, 96, 300]
    spans = [(380, 470), (10, 70), (0, 0)]
    q, k, v = _inputs(device, dtype, q_lens, k_lens, 8, 2, dqk, dv, seed=dqk + (window or 0))
    aux = [_image_ranges(q_lens, k_lens, spans, device), offsets(q_lens, device)]
    kw = dict(_NONE, cu_seqlens_q=offsets(q_lens, device), cu_seqlens_k=offsets(k_lens, device),
              max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), mask_mod=mm_prefix_mask(window, clamp),
              aux_tensors=aux)
    _check(device, q, k, v, dtype, f"mm_prefix W={window} clamp={clamp} d={dqk}/{dv}", **kw)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dqk,dv", DIMS)
@pytest.mark.parametrize("prefix,window", [(0, 64), (40, 100), (300, 16), (40, 1000)])
def test_rswa_mask(device, dtype, dqk, dv, prefix, window):
    """Rolling window with a prefix of global keys; (40, 100) over 1100 keys
    runs the prefix and the windows as two key passes."""
    q_lens, k_lens = [256, 130, 1], [1100, 700, 90]
    q, k, v = _inputs(device, dtype, q_lens, k_lens, 8, 2, dqk, dv, seed=7 * prefix + window)
    aux = [torch.tensor([prefix] * len(q_lens), dtype=torch.int32, device=device),
           torch.tensor([window], dtype=torch.int32, device=device)]
    kw = dict(_NONE, cu_seqlens_q=offsets(q_lens, device), cu_seqlens_k=offsets(k_lens, device),
              max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), mask_mod=rswa_mask(), aux_tensors=aux)
    _check(device, q, k, v, dtype, f"rswa P={prefix} W={window} d={dqk}/{dv}", **kw)


@pytest.mark.parametrize("mask_name", ["prefix", "prefix clamped", "rolling window"])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (16, 8), (6, 2)])
@pytest.mark.parametrize("page", [16, 64])
def test_masks_over_pages_and_head_groups(device, mask_name, hq, hkv, page):
    """Paged K/V (NaN-poisoned free slots), one query head a workgroup (odd
    groups) or two, per-request prefixes."""
    dtype, d = torch.bfloat16, 128
    q_lens, k_lens = [150, 64, 300], [650, 64, 300]
    q, k, v = _inputs(device, dtype, q_lens, k_lens, hq, hkv, d, d, seed=hq * page)
    kc, vc, table = _paged(k, v, k_lens, page, device, seed=page)
    if mask_name == "rolling window":
        mask = rswa_mask()
        aux = [torch.tensor([20, 0, 129], dtype=torch.int32, device=device),
               torch.tensor([75], dtype=torch.int32, device=device)]
    else:
        mask = mm_prefix_mask(None if mask_name == "prefix" else 90, mask_name == "prefix clamped")
        aux = [_image_ranges(q_lens, k_lens, [(520, 600), (0, 64), (100, 250)], device), offsets(q_lens, device)]
    kw = dict(_NONE, cu_seqlens_q=offsets(q_lens, device), cu_seqlens_k=None,
              seqused_k=torch.tensor(k_lens, dtype=torch.int32, device=device), block_table=table,
              max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), mask_mod=mask, aux_tensors=aux)
    _check(device, q, kc, vc, dtype, f"{mask_name} paged P={page} {hq}/{hkv}", **kw)


@pytest.mark.parametrize("d,cap", [(128, 30.0), (256, 30.0), (256, 0.0)])
@pytest.mark.parametrize("mask_name", ["prefix+window", "rolling window"])
def test_masks_with_fp8_cache_and_softcap(device, mask_name, d, cap):
    """E4M3 K/V with per-(request, KV head) descales, with and without
    softcap 30 (256-dim heads: the V-half tile)."""
    dtype, fp8 = torch.bfloat16, torch.float8_e4m3fn
    q_lens, k_lens = [100, 250], [400, 250]
    q, k, v = _inputs(device, dtype, q_lens, k_lens, 8, 2, d, d, seed=41 + d)
    k8, v8 = (k * 4).to(fp8), (v * 4).to(fp8)
    kd = torch.full((2, 2), 0.25, device=device)
    if mask_name == "rolling window":
        mask, aux = rswa_mask(), [torch.tensor([10, 30], dtype=torch.int32, device=device),
                                  torch.tensor([50], dtype=torch.int32, device=device)]
    else:
        mask = mm_prefix_mask(64)
        aux = [_image_ranges(q_lens, k_lens, [(320, 390), (20, 100)], device), offsets(q_lens, device)]
    kw = dict(_NONE, cu_seqlens_q=offsets(q_lens, device), cu_seqlens_k=offsets(k_lens, device),
              max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), mask_mod=mask, aux_tensors=aux, softcap=cap,
              k_descale=kd, v_descale=kd)
    _check(device, q, k8, v8, dtype, f"{mask_name} E4M3 K/V d={d} cap={cap}", **kw)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("cap", [512, 600, 1000])
def test_cache_leftpad_on_the_mfma_prefill(device, dtype, d, causal, cap):
    """flash_attn_with_kvcache over a dense cache with cache_leftpad: key j
    of request b sits at slot leftpad[b] + j.  Capacities that are not powers
    of two run as one page per request (every position in page 0)."""
    batch, sq, hq, hkv = 3, 40, 8, 2
    g = torch.Generator().manual_seed(d)
    q = (torch.randn(batch, sq, hq, d, generator=g) * 0.5).to(dtype).to(device)
    kc = (torch.randn(batch, cap, hkv, d, generator=g) * 0.5).to(dtype).to(device)
    vc = (torch.randn(batch, cap, hkv, d, generator=g) * VALUE_SCALE).to(dtype).to(device)
    seqlens = torch.tensor([min(500, cap), 300, 77], dtype=torch.int32, device=device)
    leftpad = torch.tensor([13, 0, 30], dtype=torch.int32, device=device)
    out, lse = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens, cache_leftpad=leftpad, causal=causal,
                                       return_softmax_lse=True)
    # The same call's kernel arguments: a one-page-per-request table.
    lengths = seqlens - leftpad
    table = torch.arange(batch, dtype=torch.int32, device=device).reshape(batch, 1)
    cuq = offsets([sq] * batch, device)
    probe = torch.empty(batch * sq, hq, d, dtype=dtype, device=device)
    keep = []
    args = kernel_args(q.flatten(0, 1), kc, vc, probe, torch.empty(hq, batch * sq, device=device), keep=keep,
                       **dict(_NONE, cu_seqlens_q=cuq, cu_seqlens_k=None, seqused_k=lengths, block_table=table,
                              max_seqlen_q=sq, max_seqlen_k=cap, causal=causal, leftpad_k=leftpad,
                              mask_mod=None, aux_tensors=None))
    assert _lib.supported("fa_prefill_supported", args)
    ref, ref_lse = oracle_attention(q.flatten(0, 1), kc, vc, cuq, used_k=lengths, block_table=table,
                                    leftpad=leftpad, causal=causal)
    assert_parity(out.flatten(0, 1), lse.permute(1, 0, 2).reshape(hq, -1), ref, ref_lse, dtype)
