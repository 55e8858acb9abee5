"""256-dim MFMA prefill run as two V-column halves vs the fp64 oracle.

fa_prefill_fwd runs 256-dim heads as two workgroups per work item, one per
128-column half of V and of the output (prefill_vparts in
prefill_kernel.h; the one-pass 256/256 tile stays for 16-bit softcaps and for
E4M3 softcaps with a window).  Both halves recompute S; only the first
writes the LSE.  These cases pin the part decoding against both work-list
modes (compact up to 256 requests, the per-pair grid beyond), one and two
query heads per workgroup, strided V and output views (the second half's
columns start DVT elements into the row, whatever the strides), spare
output rows and columns that must stay unwritten, and E4M3 K/V on both
routes.  Bar: this build's (max-abs <= 1e-2 bf16, LSE <= 1e-4) on rows that
see at least 32 keys, plus the all-rows check of assert_parity.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib, vllm
from harness import assert_parity, attention, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu

VALUE_SCALE = 0.5
E4M3 = torch.float8_e4m3fn


def _route_mfma(q, k, v, **kw):
    keep = []
    out = torch.empty(q.shape[0], q.shape[1], v.shape[-1], dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[1], q.shape[0], device=q.device)
    full = dict(cu_seqlens_q=None, cu_seqlens_k=None, seqused_k=None, max_seqlen_q=1, max_seqlen_k=1,
                block_table=None, softmax_scale=None, causal=False, window_size=(-1, -1), alibi_slopes=None,
                softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None, mask_mod=None,
                aux_tensors=None, leftpad_k=None)
    full.update(kw)
    return _lib.supported("fa_prefill_supported", kernel_args(q, k, v, out, lse, keep=keep, **full))


def _many_key_rows(q_lens, k_lens, causal=True):
    rows, start = [], 0
    for n, m in zip(q_lens, k_lens):
        rows += [start + i for i in range(n) if (m - n + i + 1 if causal else m) >= 32]
        start += n
    return torch.tensor(rows)


@pytest.mark.parametrize("batch,hq,hkv", [(9, 16, 8), (9, 16, 16), (20, 12, 4), (13, 6, 2), (257, 8, 2)])
def test_d256_halves_work_list_modes(device, batch, hq, hkv):
    """Compact work list (batch <= 256) and the per-pair grid (257), with
    GQA groups 2 (two heads a workgroup), 1 and 3 (one head a workgroup);
    empty and one-row requests; spare query rows stay NaN."""
    g = torch.Generator().manual_seed(batch * 10 + hq + hkv)
    q_lens = torch.randint(0, 160, (batch,), generator=g)
    q_lens[::7] = 0
    q_lens[1::5] = 1
    k_lens = (q_lens + torch.randint(0, 90, (batch,), generator=g)).tolist()
    q_lens = q_lens.tolist()
    spare = 40
    q = (torch.randn(sum(q_lens) + spare, hq, 256, generator=g) * 0.5).to(torch.bfloat16).to(device)
    k = (torch.randn(sum(k_lens), hkv, 256, generator=g) * 0.5).to(torch.bfloat16).to(device)
    v = (torch.randn(sum(k_lens), hkv, 256, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
    cuq, cuk = offsets(q_lens, device), offsets(k_lens, device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), causal=True)
    assert _route_mfma(q, k, v, **kw)
    out = torch.full_like(q, float("nan"))
    out, lse = attention(q, k, v, out=out, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True)
    rows = torch.arange(sum(q_lens))
    assert_parity(out[rows], lse[:, rows], ref[rows], ref_lse[:, rows], torch.bfloat16)
    many = _many_key_rows(q_lens, k_lens)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=many)
    assert torch.isnan(out[sum(q_lens):].float()).all(), "spare rows past the last request were written"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal,window,alibi", [(True, (-1, -1), False), (False, (100, 30), False),
                                                 (True, (-1, -1), True), (True, (60, 0), True)])
def test_d256_halves_strided_views(device, dtype, causal, window, alibi):
    """K and V interleaved per head in one buffer (head stride 512, V offset
    by 256 elements) and an output view with 320-element head rows: each
    half reads its 128 V columns and writes its 128 output columns, and the
    64 columns past the head stay NaN."""
    g = torch.Generator().manual_seed(int(causal) + 7 * window[0] + int(alibi))
    q_lens, k_lens = [1, 77, 300, 129], [40, 77, 520, 129]
    hq, hkv = 8, 4
    q = (torch.randn(sum(q_lens), hq, 256, generator=g) * 0.5).to(dtype).to(device)
    kv = torch.randn(sum(k_lens), hkv, 2, 256, generator=g)
    kv[:, :, 1] *= VALUE_SCALE
    kv = kv.to(dtype).to(device)
    k, v = kv[:, :, 0], kv[:, :, 1]
    assert k.stride(1) == 512 and v.stride(1) == 512
    slopes = (2.0 ** (-8.0 * torch.arange(1, hq + 1) / hq)).float().to(device) if alibi else None
    cuq, cuk = offsets(q_lens, device), offsets(k_lens, device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=causal, window_size=window, alibi_slopes=slopes)
    assert _route_mfma(q, k, v, **kw)
    wide = torch.full((sum(q_lens), hq, 320), float("nan"), dtype=dtype, device=device)
    out, lse = attention(q, k, v, out=wide[..., :256], **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal, window=window,
                                    alibi=None if slopes is None else slopes.cpu())
    assert_parity(out, lse, ref, ref_lse, dtype)
    assert torch.isnan(wide[..., 256:].float()).all(), "columns past the head were written"


def _fp8_case(device, q_lens, k_lens, hq, hkv, seed):
    g = torch.Generator().manual_seed(seed)
    b = len(q_lens)
    ks = torch.empty(b, hkv).uniform_(0.02, 0.2, generator=g)
    vs = torch.empty(b, hkv).uniform_(0.02, 0.2, generator=g)
    per_tok = lambda s: torch.cat([s[i].expand(n, hkv) for i, n in enumerate(k_lens)])[..., None]
    q = (torch.randn(sum(q_lens), hq, 256, generator=g) * 2.0).to(torch.bfloat16).to(device)
    k = (torch.randn(sum(k_lens), hkv, 256, generator=g) * 0.5 / per_tok(ks)).to(E4M3).to(device)
    v = (torch.randn(sum(k_lens), hkv, 256, generator=g) * VALUE_SCALE / per_tok(vs)).to(E4M3).to(device)
    return q, k, v, ks.to(device), vs.to(device)


@pytest.mark.parametrize("cap,window", [(0.0, (-1, -1)), (30.0, (-1, -1)), (0.0, (127, 0)), (30.0, (127, 0))])
def test_d256_e4m3_both_routes(device, cap, window):
    """E4M3 K/V with per-(request, KV head) descales: V halves without a
    softcap or without a window, the one-pass tile for a softcap with a
    window; sinks on every case."""
    q_lens, k_lens = [3, 129, 300, 64], [40, 129, 300, 600]
    hq, hkv = 16, 8
    q, k, v, ks, vs = _fp8_case(device, q_lens, k_lens, hq, hkv, seed=int(cap) + window[0])
    sinks = torch.randn(hq, generator=torch.Generator().manual_seed(3)).to(device)
    cuq, cuk = offsets(q_lens, device), offsets(k_lens, device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=True, window_size=window, softcap=cap, s_aux=sinks, k_descale=ks, v_descale=vs)
    assert _route_mfma(q, k, v, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, window=window, softcap=cap,
                                    sinks=sinks.cpu(), k_descale=ks, v_descale=vs)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_d256_halves_paged_mixed_batch(device):
    """Paged 256-dim caches in a mixed chunked-prefill + decode batch through
    the vLLM contract (q_len 1 requests on the decode kernel, the rest on the
    V-half prefill)."""
    g = torch.Generator().manual_seed(256)
    page, hq, hkv, d = 16, 8, 2, 256
    q_lens, k_lens = [1, 300, 1, 77, 2, 129], [900, 700, 33, 77, 2, 1000]
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens)
    table = torch.randperm(pool, generator=g).int().reshape(len(k_lens), cols)
    kc = (torch.randn(pool, page, hkv, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    vc = (torch.randn(pool, page, hkv, d, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    out, lse = vllm.flash_attn_varlen_func(q, kc, vc, max(q_lens), cuq, cols * page, seqused_k=used,
                                           block_table=table.to(device), causal=True, return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=True)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=_many_key_rows(q_lens, k_lens))


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, E4M3])
def test_d256_halves_requests_alone_and_batched(device, kv_dtype):
    """Each request's rows are bit-identical whether it runs alone or in a
    batch (the work list and the halves change, a row's arithmetic does not).
    Every request has two or more query rows: single-query requests take the
    decode kernel, whose default split plan depends on the batch (its
    fixed-order route is the batch-invariant one, tested elsewhere)."""
    g = torch.Generator().manual_seed(2560)
    q_lens, k_lens = [300, 2, 129, 700, 64], [300, 40, 129, 900, 64]
    hq, hkv = 16, 8
    q = (torch.randn(sum(q_lens), hq, 256, generator=g) * 0.5).to(torch.bfloat16).to(device)
    k = (torch.randn(sum(k_lens), hkv, 256, generator=g) * 0.5).to(kv_dtype).to(device)
    v = (torch.randn(sum(k_lens), hkv, 256, generator=g) * VALUE_SCALE).to(kv_dtype).to(device)
    cuq, cuk = offsets(q_lens, device), offsets(k_lens, device)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens),
                         max_seqlen_k=max(k_lens), causal=True)
    qo, ko = 0, 0
    for i, (n, m) in enumerate(zip(q_lens, k_lens)):
        one_q, one_k = offsets([n], device), offsets([m], device)
        o1, l1 = attention(q[qo:qo + n], k[ko:ko + m], v[ko:ko + m], cu_seqlens_q=one_q, cu_seqlens_k=one_k,
                           max_seqlen_q=n, max_seqlen_k=m, causal=True)
        assert torch.equal(o1, out[qo:qo + n]), f"request {i}: output"
        assert torch.equal(l1, lse[:, qo:qo + n]), f"request {i}: LSE"
        qo, ko = qo + n, ko + m
