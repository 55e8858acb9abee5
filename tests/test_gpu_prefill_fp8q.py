"""MFMA prefill with E4M3 queries over E4M3 K/V vs the fp64 oracle.

FP8 queries are part of the reference's dtype contract (flash_attn_mps/
_attention.py:17-20 maps float8_e4m3fn for every operand; :120 makes the
output fp16 unless the caller's `out` says otherwise).  On gfx950 the scores come
from v_mfma_f32_32x32x64_f8f6f4: E4M3 x E4M3 products are exact in fp32 and
the dot is accumulated in fp32, so S carries the same error as the 16-bit
path; q_descale * k_descale joins the softmax scale and v_descale scales the
output (flash_attn_mps/kernels/attention.metal:47-51, 170-180).  V is widened
exactly to the output's 16-bit type for P.V.  Bars, on every row: max-abs
<= 1e-2 bf16 / 2e-3 fp16, LSE <= 1e-4 (-inf where a row sees no key).
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from harness import assert_parity, attention, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu

E4M3 = torch.float8_e4m3fn

# Every finite E4M3FN code: all bytes but 0x7F and 0xFF (the NaNs).
FINITE_CODES = torch.tensor([c for c in range(256) if c & 0x7F != 0x7F], dtype=torch.uint8)



def _route_is_mfma(q, k, v, out_dtype, **kw):
    keep = []
    out = torch.empty(q.shape[0], q.shape[1], v.shape[-1], dtype=out_dtype, device=q.device)
    lse = torch.empty(q.shape[1], q.shape[0], device=q.device)
    full = dict(cu_seqlens_q=None, cu_seqlens_k=None, seqused_k=None, max_seqlen_q=1, max_seqlen_k=1,
                block_table=None, softmax_scale=None, causal=False, window_size=(-1, -1), alibi_slopes=None,
                softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None, mask_mod=None,
                aux_tensors=None, leftpad_k=None)
    full.update(kw)
    return _lib.supported("fa_prefill_supported", kernel_args(q, k, v, out, lse, keep=keep, **full))


def _e4m3(x):
    """Saturating E4M3 quantisation (torch's cast turns |x| > 448 into NaN)."""
    return x.clamp(-448.0, 448.0).to(E4M3)


def _descales(g, batch, hkv, device, lo, hi):
    return torch.empty(batch, hkv).uniform_(lo, hi, generator=g).to(device)


def _packed(device, d, hq, hkv, q_lens, k_lens, seed, qscale=0.5, vscale=0.5):
    """E4M3 q/k/v quantised with per-(request, KV head) scales; returns the
    codes and the descales that restore them."""
    g = torch.Generator().manual_seed(seed)
    b = len(q_lens)
    qs = _descales(g, b, hkv, "cpu", 0.005, 0.02)
    ks = _descales(g, b, hkv, "cpu", 0.005, 0.02)
    vs = _descales(g, b, hkv, "cpu", 0.005, 0.02)
    group = hq // hkv

    def per_token(s, lens, heads_per):
        return torch.cat([s[i].repeat_interleave(heads_per).expand(n, -1) for i, n in enumerate(lens)])[..., None]

    q = _e4m3(torch.randn(sum(q_lens), hq, d, generator=g) * qscale / per_token(qs, q_lens, group))
    k = _e4m3(torch.randn(sum(k_lens), hkv, d, generator=g) * 0.5 / per_token(ks, k_lens, 1))
    v = _e4m3(torch.randn(sum(k_lens), hkv, d, generator=g) * vscale / per_token(vs, k_lens, 1))
    return (q.to(device), k.to(device), v.to(device), qs.to(device), ks.to(device), vs.to(device),
            offsets(q_lens, device), offsets(k_lens, device))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_fp8q_prefill_packed(device, out_dtype, d, causal):
    q_lens, k_lens = [1, 37, 300, 64, 513], [5, 37, 300, 200, 700]
    q, k, v, qs, ks, vs, cuq, cuk = _packed(device, d, 8, 2, q_lens, k_lens, seed=d + causal)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=causal, q_descale=qs, k_descale=ks, v_descale=vs)
    assert _route_is_mfma(q, k, v, out_dtype, **kw)
    out = torch.empty(q.shape[0], 8, d, dtype=out_dtype, device=device)
    out, lse = attention(q, k, v, out=out, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal, q_descale=qs, k_descale=ks, v_descale=vs)
    assert_parity(out, lse, ref, ref_lse, out_dtype)


def test_fp8q_default_output_is_fp16(device):
    """With no `out`, E4M3 queries produce fp16 (the reference's rule)."""
    q, k, v, qs, ks, vs, cuq, cuk = _packed(device, 128, 4, 4, [200], [200], seed=11)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=200, max_seqlen_k=200,
                         causal=True, q_descale=qs, k_descale=ks, v_descale=vs)
    assert out.dtype == torch.float16
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, q_descale=qs, k_descale=ks, v_descale=vs)
    assert_parity(out, lse, ref, ref_lse, torch.float16)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_fp8q_all_finite_codes(device, d):
    """Known-answer case: Q, K and V each hold every one of the 254 finite
    E4M3 codes (subnormals, both zeros, +-448) at many positions, through
    the MFMA route.  Descales of 2^-8 keep the scores and outputs O(1)."""
    hq, hkv, n = 4, 2, 254
    count = lambda heads: n * heads * d

    def tile(shift, heads):
        idx = (torch.arange(count(heads)) * 7 + shift) % FINITE_CODES.numel()
        return FINITE_CODES[idx].view(E4M3).reshape(n, heads, d)

    q, k, v = tile(0, hq).to(device), tile(3, hkv).to(device), tile(101, hkv).to(device)
    for t in (q, k, v):
        seen = torch.unique(t.view(torch.uint8).cpu())
        assert seen.numel() == 254 and not bool(((seen & 0x7F) == 0x7F).any())
    desc = torch.full((1, hkv), 2.0 ** -8, device=device)
    vdesc = torch.full((1, hkv), 1.0 / 448, device=device)
    cu = offsets([n], device)
    for out_dtype in (torch.bfloat16, torch.float16):
        for causal in (True, False):
            kw = dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=n, max_seqlen_k=n, causal=causal,
                      q_descale=desc, k_descale=desc, v_descale=vdesc)
            assert _route_is_mfma(q, k, v, out_dtype, **kw)
            out = torch.empty(n, hq, d, dtype=out_dtype, device=device)
            out, lse = attention(q, k, v, out=out, **kw)
            ref, ref_lse = oracle_attention(q, k, v, cu, cu, causal=causal, q_descale=desc, k_descale=desc,
                                            v_descale=vdesc)
            assert_parity(out, lse, ref, ref_lse, out_dtype, what=f"d{d} {out_dtype} causal={causal}")


@pytest.mark.parametrize("page", [16, 256])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_fp8q_prefill_paged_poisoned_tail(device, page, d):
    """Paged E4M3 caches through a permuted block table; every slot past a
    request's length holds the E4M3 NaN code and must never be read."""
    g = torch.Generator().manual_seed(page * 3 + d)
    hq, hkv = 8, 2
    q_lens, k_lens = [300, 33, 129, 1], [700, 33, 1029, 517]
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens) + 2
    table = torch.randperm(pool, generator=g)[:cols * len(k_lens)].int().reshape(len(k_lens), cols)
    ks = _descales(g, len(k_lens), hkv, "cpu", 0.005, 0.02)
    vs = _descales(g, len(k_lens), hkv, "cpu", 0.005, 0.02)
    qs = _descales(g, len(k_lens), hkv, "cpu", 0.005, 0.02)
    kq = torch.full((pool, page, hkv, d), float("nan")).to(E4M3)
    vq = torch.full((pool, page, hkv, d), float("nan")).to(E4M3)
    for b, n in enumerate(k_lens):
        pos = torch.arange(n)
        pages, slots = table[b, pos // page].long(), pos % page
        kq[pages, slots] = _e4m3(torch.randn(n, hkv, d, generator=g) * 0.5 / ks[b][:, None])
        vq[pages, slots] = _e4m3(torch.randn(n, hkv, d, generator=g) * 0.5 / vs[b][:, None])
    group = hq // hkv
    qdiv = torch.cat([qs[b].repeat_interleave(group).expand(n, -1) for b, n in enumerate(q_lens)])[..., None]
    q = _e4m3(torch.randn(sum(q_lens), hq, d, generator=g) * 0.5 / qdiv).to(device)
    kq, vq, qs, ks, vs = kq.to(device), vq.to(device), qs.to(device), ks.to(device), vs.to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    kw = dict(cu_seqlens_q=cuq, seqused_k=used, max_seqlen_q=max(q_lens), max_seqlen_k=cols * page,
              block_table=table.to(device), causal=True, q_descale=qs, k_descale=ks, v_descale=vs)
    assert _route_is_mfma(q, kq, vq, torch.bfloat16, **kw)
    out = torch.empty(q.shape[0], hq, d, dtype=torch.bfloat16, device=device)
    out, lse = attention(q, kq, vq, out=out, **kw)
    assert torch.isfinite(out).all()
    ref, ref_lse = oracle_attention(q, kq, vq, cuq, used_k=used, block_table=table, causal=True,
                                    q_descale=qs, k_descale=ks, v_descale=vs)
    assert_parity(out, None, ref, None, torch.bfloat16)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("window", [(-1, -1), (127, 0), (40, -1)])
@pytest.mark.parametrize("cap", [0.0, 30.0])
def test_fp8q_prefill_softcap_window_sinks(device, window, cap, d):
    """Softcap, windows and sinks; 256-dim heads run as two V-column halves."""
    q_lens, k_lens = [3, 129, 300, 64], [40, 129, 300, 600]
    q, k, v, qs, ks, vs, cuq, cuk = _packed(device, d, 8, 2, q_lens, k_lens, seed=int(cap) + window[0] + 50 + d,
                                            qscale=2.0)
    assert not torch.isnan(q.float()).any()
    sinks = torch.randn(8, generator=torch.Generator().manual_seed(3)).to(device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=True, window_size=window, softcap=cap, s_aux=sinks, q_descale=qs, k_descale=ks,
              v_descale=vs)
    assert _route_is_mfma(q, k, v, torch.bfloat16, **kw)
    out = torch.empty(q.shape[0], 8, d, dtype=torch.bfloat16, device=device)
    out, lse = attention(q, k, v, out=out, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, window=window, softcap=cap,
                                    sinks=sinks.cpu(), q_descale=qs, k_descale=ks, v_descale=vs)
    assert_parity(out, None, ref, None, torch.bfloat16)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_fp8q_mixed_batch_with_single_query_requests(device):
    """Chunked prefill + decode rows in one batch over a paged E4M3 cache."""
    g = torch.Generator().manual_seed(91)
    page, hq, hkv, d = 16, 16, 8, 128
    q_lens = [1, 300, 1, 77, 1, 2]
    k_lens = [900, 700, 4000, 77, 33, 2]
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens)
    table = torch.randperm(pool, generator=g).int().reshape(len(k_lens), cols).to(device)
    scale = torch.empty(hkv).uniform_(0.005, 0.02, generator=g)
    kc = _e4m3(torch.randn(pool, page, hkv, d, generator=g) * 0.5 / scale[:, None]).to(device)
    vc = _e4m3(torch.randn(pool, page, hkv, d, generator=g) * 0.5 / scale[:, None]).to(device)
    desc = scale.to(device).expand(len(k_lens), hkv)
    q = _e4m3(torch.randn(sum(q_lens), hq, d, generator=g) * 0.5 / 0.01).to(device)
    qdesc = torch.full((len(k_lens), hkv), 0.01, device=device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    out = torch.full((sum(q_lens), hq, d), float("nan"), dtype=torch.bfloat16, device=device)
    out, lse = attention(q, kc, vc, cu_seqlens_q=cuq, seqused_k=used, max_seqlen_q=max(q_lens),
                         max_seqlen_k=cols * page, block_table=table, causal=True, q_descale=qdesc,
                         k_descale=desc, v_descale=desc, out=out)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=True,
                                    q_descale=qdesc, k_descale=desc, v_descale=desc)
    assert_parity(out, None, ref, None, torch.bfloat16)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_fp8q_unsupported_dims_take_the_generic_kernel(device):
    """E4M3 queries at a head dim the MFMA kernel does not compile (96)."""
    q, k, v, qs, ks, vs, cuq, cuk = _packed(device, 96, 4, 2, [70], [70], seed=1)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=70, max_seqlen_k=70, causal=True,
              q_descale=qs, k_descale=ks, v_descale=vs)
    assert not _route_is_mfma(q, k, v, torch.float16, **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, q_descale=qs, k_descale=ks, v_descale=vs)
    assert_parity(out, lse, ref, ref_lse, torch.float16)


def test_fp8q_negative_scale_and_descales(device):
    """E4M3 queries with a negative softmax_scale and negative q descales on
    some (request, KV head) pairs: each workgroup's score scale takes its own
    sign, and the row max is that of the scaled scores."""
    q_lens, k_lens = [37, 300, 513], [37, 400, 700]
    q, k, v, qs, ks, vs, cuq, cuk = _packed(device, 128, 8, 2, q_lens, k_lens, seed=77, qscale=2.0)
    qs = qs.clone()
    qs[0, 1] *= -1
    qs[2, 0] *= -1
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=True, softmax_scale=-(128 ** -0.5), q_descale=qs, k_descale=ks, v_descale=vs)
    assert _route_is_mfma(q, k, v, torch.bfloat16, **kw)
    out = torch.empty(q.shape[0], 8, 128, dtype=torch.bfloat16, device=device)
    out, lse = attention(q, k, v, out=out, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, scale=-(128 ** -0.5), q_descale=qs,
                                    k_descale=ks, v_descale=vs)
    assert torch.isfinite(out).all()
    assert_parity(out, None, ref, None, torch.bfloat16)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
