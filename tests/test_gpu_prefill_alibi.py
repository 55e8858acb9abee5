"""ALiBi on the MFMA prefill kernel vs the fp64 oracle.

The bias -slope * |q_pos + k_len - q_len - k_pos| is added to the scaled
score (flash_attn_mps/_attention.py applies it after softcap; the oracle in
oracle/attention.py:109-112 restates that).  Covered: causal and non-causal,
per-head [Hq] and per-request [B, Hq] slopes, GQA with and without head
packing, packed and paged K/V, q_len != k_len, sinks, BLOOM-sized slopes on
long keys, ALiBi after a softcap, with windows, per-request causality and
E4M3 K/V (64/128/256-dim heads, E4M3 K/V too), negative and zero score
scales, and that the MFMA kernel is the route taken (padded head dims keep
the combinations on the generic kernel).  Tolerances: max-abs <= 2e-3 fp16,
<= 1e-2 bf16, LSE <= 1e-4.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from harness import assert_parity, attention, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu


def _route(q, k, v, **kw):
    """True when fa_prefill_fwd accepts the call."""
    out = torch.empty(q.shape[0], q.shape[1], v.shape[-1], dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[1], q.shape[0], device=q.device)
    full = dict(cu_seqlens_q=None, cu_seqlens_k=None, seqused_k=None, max_seqlen_q=1, max_seqlen_k=1,
                block_table=None, softmax_scale=None, causal=False, window_size=(-1, -1), alibi_slopes=None,
                softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None, mask_mod=None,
                aux_tensors=None, leftpad_k=None)
    full.update(kw)
    keep = []
    return _lib.supported("fa_prefill_supported", kernel_args(q, k, v, out, lse, keep=keep, **full))


def _case(device, dtype, d, hq, hkv, q_lens, k_lens, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(dtype).to(device)
    k = (torch.randn(sum(k_lens), hkv, d, generator=g) * 0.5).to(dtype).to(device)
    v = torch.randn(sum(k_lens), hkv, d, generator=g).to(dtype).to(device)
    return q, k, v, offsets(q_lens, device), offsets(k_lens, device)


def _bloom_slopes(heads):
    """Geometric slopes 2^(-8 i / heads), i = 1..heads (the ALiBi paper's schedule)."""
    return torch.tensor([2.0 ** (-8.0 * (i + 1) / heads) for i in range(heads)])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_alibi_prefill(device, dtype, d, causal):
    q_lens, k_lens = [1, 37, 300, 64, 513], [5, 37, 300, 200, 700]
    q, k, v, cuq, cuk = _case(device, dtype, d, 8, 2, q_lens, k_lens, seed=d + causal)
    slopes = _bloom_slopes(8).to(device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=causal, alibi_slopes=slopes)
    assert _route(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal, alibi=slopes)
    assert_parity(out, lse, ref, ref_lse, dtype)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 8), (12, 4), (8, 1)])
def test_alibi_per_request_slopes_gqa(device, hq, hkv):
    """[B, Hq] slopes: each request and head has its own slope (odd groups skip head packing)."""
    q_lens = [129, 256, 1000]
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, hq, hkv, q_lens, q_lens, seed=hq * 7 + hkv)
    g = torch.Generator().manual_seed(hq)
    slopes = (torch.rand(len(q_lens), hq, generator=g) * 0.3).to(device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=1000, max_seqlen_k=1000, causal=True,
              alibi_slopes=slopes)
    assert _route(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, alibi=slopes)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_alibi_long_keys_steep_slopes(device):
    """Slopes up to 0.5 over 2048 keys: biases reach -1000, far below any score.

    Steep slopes leave a few keys with nearly all the weight, so an output is
    close to one value row; V is scaled by 1/4 to keep outputs below 2, where
    bf16's own rounding of the output (half an ulp, <= 2^-8) stays inside the
    1e-2 bar (a row of 4 would round by up to 1.6e-2 in any bf16 kernel).
    """
    q_lens, k_lens = [2048, 100], [2048, 1500]
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, 8, 8, q_lens, k_lens, seed=5)
    v = v * 0.25
    slopes = _bloom_slopes(8).to(device)
    for causal in (True, False):
        out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=2048,
                             max_seqlen_k=2048, causal=causal, alibi_slopes=slopes)
        ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal, alibi=slopes)
        assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


@pytest.mark.parametrize("page", [16, 128])
def test_alibi_paged_with_sinks(device, page):
    g = torch.Generator().manual_seed(page)
    k_lens, q_lens = [700, 33, 1029], [300, 33, 129]
    hq, hkv, d = 8, 4, 128
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens) + 3
    table = torch.randperm(pool, generator=g)[:cols * len(k_lens)].int().reshape(len(k_lens), cols)
    kc = (torch.randn(pool, page, hkv, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    vc = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16).to(device)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    table = table.to(device)
    slopes = _bloom_slopes(hq).to(device)
    sinks = torch.linspace(-1.0, 2.0, hq).to(device)
    kw = dict(cu_seqlens_q=cuq, seqused_k=used, max_seqlen_q=max(q_lens), max_seqlen_k=cols * page,
              block_table=table, causal=True, alibi_slopes=slopes, s_aux=sinks)
    assert _route(q, kc, vc, **kw)
    out, lse = attention(q, kc, vc, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=True,
                                       alibi=slopes, sinks=sinks)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


COMBOS = ["softcap", "window", "softcap+window", "per-request causal", "fp8", "fp8+softcap+window"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,extra", [(d, e) for d in (64, 128, 256) for e in COMBOS])
def test_alibi_combinations_on_the_mfma_prefill(device, dtype, d, extra):
    """ALiBi after a softcap (softcap(score) - slope |diff|), with left / right
    windows, per-request causality and E4M3 K/V with descales
    (kernels/attention.metal:47-51, 84-87; the reference applies the bias in
    every kernel).  E4M3 K/V take it at every head dim (256: the V-half
    tile, also with a softcap and a window)."""
    q_lens, k_lens = [70, 300, 1], [200, 300, 40]
    q, k, v, cuq, cuk = _case(device, dtype, d, 8, 2, q_lens, k_lens, seed=d + len(extra))
    v = v * 0.5
    slopes = _bloom_slopes(8).to(device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=True, alibi_slopes=slopes)
    ref_kw = dict(causal=True, alibi=slopes)
    if "softcap" in extra:
        kw["softcap"] = ref_kw["softcap"] = 5.0
    if "window" in extra:
        kw["causal"] = ref_kw["causal"] = False
        kw["window_size"] = ref_kw["window"] = (48, 16)
    if extra == "per-request causal":
        flags = torch.tensor([True, False, True], device=device)
        kw["causal"], ref_kw["causal"] = flags, flags
    if extra.startswith("fp8"):
        k, v = (k * 4).to(torch.float8_e4m3fn), (v * 4).to(torch.float8_e4m3fn)
        desc = torch.full((3, 2), 0.25, device=device)
        kw["k_descale"] = kw["v_descale"] = ref_kw["k_descale"] = ref_kw["v_descale"] = desc
    assert _route(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, **ref_kw)
    assert_parity(out, lse, ref, ref_lse, dtype)


@pytest.mark.parametrize("scale", [-0.09, 0.0])
@pytest.mark.parametrize("cap", [0.0, 5.0])
def test_alibi_with_negative_or_zero_score_scale(device, scale, cap):
    """A negative scale flips Q's signs; a zero scale leaves the scores equal
    to the biases alone (the folded bias then uses a unit scale)."""
    q_lens = [64, 200]
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, 4, 2, q_lens, q_lens, seed=13)
    v = v * 0.5
    slopes = torch.tensor([0.05, 0.1, 0.2, 0.4], device=device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=200, max_seqlen_k=200, causal=True,
              alibi_slopes=slopes, softmax_scale=scale, softcap=cap)
    assert _route(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, alibi=slopes, scale=scale, softcap=cap)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_alibi_combinations_on_padded_dims_use_generic_kernel(device):
    """Padded head dims (72 runs in the 128-dim tile) keep ALiBi with a
    softcap or window on the generic kernel; the result still matches."""
    q_lens = [70, 300]
    q, k, v, cuq, cuk = _case(device, torch.float16, 72, 4, 2, q_lens, q_lens, seed=11)
    slopes = torch.tensor([0.05, 0.1, 0.2, 0.4], device=device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=300, max_seqlen_k=300, causal=True,
              alibi_slopes=slopes, softcap=5.0)
    assert not _route(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, alibi=slopes, softcap=5.0)
    assert_parity(out, lse, ref, ref_lse, torch.float16)
