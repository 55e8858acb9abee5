"""MFMA prefill kernel (fa_prefill_fwd) vs the fp64 oracle.

Covers the fast-path feature set: bf16/fp16, head dims 64/128/256, causal and
non-causal, softcap, GQA ratios, packed and paged K/V, q_len != k_len
(lower-right causality, rows with no visible key), partial query/key tiles,
and that the MFMA path is the one taken.  Tolerances: this build's bar
(max-abs <= 2e-3 fp16, <= 1e-2 bf16, LSE <= 1e-4).
"""
import pytest
import torch

from flash_attn_mps_amd import _lib, flash_attn_varlen_func, vllm
from harness import assert_parity, attention, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu

# Values are 0.5*N(0,1), as in benchmark config 2: the MFMA kernels round the
# softmax weights to 16 bits before P.V, which bounds a row's error by about
# 2^-8 max|v| (bf16) or 2^-10 max|v| (fp16); at this scale that stays under
# the parity bar with room, as config 2 does on every row.
VALUE_SCALE = 0.5


def _uses_mfma(q, k, v, out, lse, **kw):
    keep = []
    a = kernel_args(q, k, v, out, lse, keep=keep, **kw)
    return _lib.supported("fa_prefill_supported", a)


def _case(device, dtype, d, hq, hkv, q_lens, k_lens, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * scale).to(dtype).to(device)
    k = (torch.randn(sum(k_lens), hkv, d, generator=g) * scale).to(dtype).to(device)
    v = (torch.randn(sum(k_lens), hkv, d, generator=g) * VALUE_SCALE).to(dtype).to(device)
    return q, k, v, offsets(q_lens, device), offsets(k_lens, device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [32, 64, 72, 80, 96, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_dims_causal(device, dtype, d, causal):
    q_lens, k_lens = [1, 37, 300, 64, 513], [5, 37, 300, 200, 700]
    q, k, v, cuq, cuk = _case(device, dtype, d, 8, 2, q_lens, k_lens, scale=0.5, seed=d)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens),
                         max_seqlen_k=max(k_lens), causal=causal)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal)
    assert_parity(out, lse, ref, ref_lse, dtype)


def test_prefill_route_is_mfma(device):
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, 16, 8, [300, 17], [300, 17])
    out = torch.empty_like(q)
    lse = torch.empty(16, q.shape[0], device=device)
    assert _uses_mfma(q, k, v, out, lse, cu_seqlens_q=cuq, cu_seqlens_k=cuk, seqused_k=None, max_seqlen_q=300,
                      max_seqlen_k=300, block_table=None, softmax_scale=None, causal=True, window_size=(-1, -1),
                      alibi_slopes=None, softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None,
                      mask_mod=None, aux_tensors=None, leftpad_k=None)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 8), (32, 8), (8, 1), (16, 2), (28, 4), (12, 2)])
def test_prefill_gqa_ratios(device, hq, hkv):
    q_lens = [129, 256, 1000]
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, hq, hkv, q_lens, q_lens, scale=0.5, seed=hq * 7 + hkv)
    out, lse = flash_attn_varlen_func(q, k, v, cuq, cuk, max(q_lens), max(q_lens), causal=True,
                                      return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True)
    # The first rows of each request see a few keys (outputs near single V
    # rows of |v| up to 4): the reference's tolerance there, this build's bar
    # on rows that see 32 keys or more.
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    rows = torch.cat([torch.arange(s + 31, s + n) for s, n in zip(cuq[:-1].tolist(), q_lens)])
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=rows)


@pytest.mark.parametrize("cap", [0.5, 5.0, 50.0])
def test_prefill_softcap(device, cap):
    q_lens, k_lens = [70, 300], [100, 300]
    q, k, v, cuq, cuk = _case(device, torch.float16, 128, 4, 2, q_lens, k_lens, scale=2.0, seed=3)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=300, max_seqlen_k=300,
                         causal=True, softcap=cap)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, softcap=cap)
    assert_parity(out, lse, ref, ref_lse, torch.float16)


@pytest.mark.parametrize("page", [16, 64, 256])
def test_prefill_paged_permuted_table(device, page):
    g = torch.Generator().manual_seed(page)
    k_lens = [700, 33, 1029]
    q_lens = [300, 33, 129]
    hq, hkv, d = 8, 4, 128
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens) + 3
    table = torch.randperm(pool, generator=g)[:cols * len(k_lens)].int().reshape(len(k_lens), cols)
    kc = torch.randn(pool, page, hkv, d, generator=g)
    vc = torch.randn(pool, page, hkv, d, generator=g) * VALUE_SCALE
    for b, n in enumerate(k_lens):       # poison every slot past the request's length
        for pos in range(n, cols * page):
            kc[table[b, pos // page], pos % page] = float("nan")
            vc[table[b, pos // page], pos % page] = float("nan")
    kc, vc = kc.to(torch.bfloat16).to(device), vc.to(torch.bfloat16).to(device)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    table = table.to(device)
    out, lse = attention(q, kc, vc, cu_seqlens_q=cuq, seqused_k=used, max_seqlen_q=max(q_lens),
                         max_seqlen_k=cols * page, block_table=table, causal=True)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=True)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_prefill_more_queries_than_keys_and_empty(device):
    # Lower-right causality: the first q_len - k_len rows see no key -> 0 / -inf.
    q_lens, k_lens = [40, 0, 100], [10, 5, 0]
    q, k, v, cuq, cuk = _case(device, torch.float16, 64, 4, 4, q_lens, k_lens, seed=9)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=100, max_seqlen_k=10,
                         causal=True)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True)
    assert_parity(out, lse, ref, ref_lse, torch.float16)
    assert torch.count_nonzero(out[40:]) == 0


def test_prefill_strided_output_and_inputs(device):
    """Caller-owned strided out (rows padded) and q/k/v views with padded rows."""
    q_lens = [200, 77]
    hq, hkv, d = 8, 2, 128
    g = torch.Generator().manual_seed(21)
    qb = torch.randn(sum(q_lens), hq + 2, d, generator=g).to(torch.bfloat16).to(device)
    kb = torch.randn(sum(q_lens), hkv + 1, d, generator=g).to(torch.bfloat16).to(device)
    vb = (torch.randn(sum(q_lens), hkv + 1, d, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
    q, k, v = qb[:, 1:hq + 1], kb[:, :hkv], vb[:, 1:]
    cu = offsets(q_lens, device)
    storage = torch.full((sum(q_lens), hq + 3, d), 7.0, dtype=torch.bfloat16, device=device)
    out = storage[:, 2:hq + 2]
    res, lse = attention(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=200, max_seqlen_k=200,
                         causal=True, out=out)
    assert res.data_ptr() == out.data_ptr()
    ref, ref_lse = oracle_attention(q, k, v, cu, cu, causal=True)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    assert torch.all(storage[:, :2] == 7.0) and torch.all(storage[:, hq + 2:] == 7.0)


def test_prefill_long_softmax_stability(device):
    torch.manual_seed(191)
    q = (torch.randn(2049, 4, 128, device=device) * 3).to(torch.float16)
    k = (torch.randn(4097, 2, 128, device=device) * 3).to(torch.float16)
    v = (torch.randn(4097, 2, 128, device=device) * VALUE_SCALE).to(torch.float16)
    cuq = torch.tensor([0, 2049], device=device, dtype=torch.int32)
    cuk = torch.tensor([0, 4097], device=device, dtype=torch.int32)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=2049, max_seqlen_k=4097,
                         causal=True)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True)
    # x3-scaled inputs make rows peaked and |out| reach ~4, where the fp16
    # half-ulp alone is ~1e-3: the reference's own tolerance applies
    # (tests/reference.py:93-96 of flash_attn_mps).
    assert_parity(out, None, ref, None)
    torch.testing.assert_close(lse.cpu().double(), ref_lse, atol=1e-4, rtol=0)


def _case_dims(device, dtype, dq, dv, hq, hkv, q_lens, k_lens, scale=0.5, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(sum(q_lens), hq, dq, generator=g) * scale).to(dtype).to(device)
    k = (torch.randn(sum(k_lens), hkv, dq, generator=g) * scale).to(dtype).to(device)
    v = (torch.randn(sum(k_lens), hkv, dv, generator=g) * VALUE_SCALE).to(dtype).to(device)
    return q, k, v, offsets(q_lens, device), offsets(k_lens, device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2)])
def test_prefill_diffkv_192_128(device, dtype, causal, hq, hkv):
    """DIFFKV head dims (Dqk 192, Dv 128) on the MFMA kernel."""
    q_lens, k_lens = [3, 129, 300, 64], [3, 200, 300, 1000]
    q, k, v, cuq, cuk = _case_dims(device, dtype, 192, 128, hq, hkv, q_lens, k_lens, seed=hq + 2 * causal)
    out = torch.empty(q.shape[0], hq, 128, dtype=dtype, device=device)
    lse = torch.empty(hq, q.shape[0], device=device)
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, seqused_k=None, max_seqlen_q=300, max_seqlen_k=1000,
              block_table=None, softmax_scale=None, causal=causal, window_size=(-1, -1), alibi_slopes=None,
              softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None, mask_mod=None,
              aux_tensors=None, leftpad_k=None)
    assert _uses_mfma(q, k, v, out, lse, **kw)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=300, max_seqlen_k=1000,
                         causal=causal)
    assert out.shape == (q.shape[0], hq, 128)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal)
    assert_parity(out, lse, ref, ref_lse, dtype)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_prefill_sinks(device, d):
    """Per-head sink logits join the denominator only (rows with no key: lse = sink)."""
    q_lens, k_lens = [50, 130, 7], [10, 130, 0]
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, d, 8, 4, q_lens, k_lens, seed=31 + d)
    sinks = torch.randn(8, generator=torch.Generator().manual_seed(d)).mul(3).to(device)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=130, max_seqlen_k=130,
                         causal=True, s_aux=sinks)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, sinks=sinks.cpu())
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    # rows of the second request that see >= 32 keys meet the 1e-2 bar
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=torch.arange(50 + 31, 180))


@pytest.mark.parametrize("dq,dv", [(128, 128), (192, 128), (64, 64)])
def test_mixed_batch_routes_single_queries_to_decode(device, dq, dv):
    """Chunked prefill + decode in one paged call: q_len == 1 requests run on
    the decode kernel, the rest on the MFMA kernel (which skips them)."""
    g = torch.Generator().manual_seed(dq + dv)
    page, hq, hkv = 16, 8, 2
    q_lens = [1, 300, 1, 1, 77, 1, 2]
    k_lens = [900, 700, 1, 4000, 77, 33, 2]
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens)
    table = torch.randperm(pool, generator=g).int().reshape(len(k_lens), cols)
    kc = torch.randn(pool, page, hkv, dq, generator=g).to(torch.bfloat16).to(device)
    vc = (torch.randn(pool, page, hkv, dv, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
    q = (torch.randn(sum(q_lens), hq, dq, generator=g) * 0.5).to(torch.bfloat16).to(device)
    sinks = torch.randn(hq, generator=g).to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    out, lse = vllm.flash_attn_varlen_func(q, kc, vc, max(q_lens), cuq, cols * page, seqused_k=used,
                                           block_table=table.to(device), causal=True, s_aux=sinks,
                                           return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=True,
                                       sinks=sinks.cpu())
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    # rows that see >= 32 keys meet the 1e-2 bar (row i of a request sees k - q + i + 1 keys)
    many, start = [], 0
    for n, m in zip(q_lens, k_lens):
        many += [start + i for i in range(n) if m - n + i + 1 >= 32]
        start += n
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=torch.tensor(many))


@pytest.mark.parametrize("batch,hq,hkv", [(64, 16, 8), (65, 16, 8), (7, 16, 16), (33, 48, 24), (20, 12, 4),
                                          (128, 16, 8), (200, 8, 8), (256, 16, 8), (257, 16, 8), (50, 16, 2),
                                          (9, 8, 1), (100, 28, 4), (257, 8, 2), (33, 12, 3), (45, 36, 12),
                                          (21, 30, 6)])
def test_prefill_work_list_modes(device, batch, hq, hkv):
    """Batches of at most 256 requests launch the compact work list (longest
    request first; one request per lane up to 64, four beyond): with
    g = gcd(Hkv, 8), each XCD owns Hkv / g KV heads and 8 / g XCDs share
    them, each taking every (8 / g)-th query block.  Larger batches take the
    per-pair grid.  Lengths include empty and
    one-row requests, and q carries spare rows past the last request."""
    g = torch.Generator().manual_seed(batch * 100 + hkv)
    q_lens = torch.randint(0, 200, (batch,), generator=g)
    q_lens[::9] = 0
    q_lens[1::11] = 1
    extra = torch.randint(0, 64, (batch,), generator=g)
    k_lens = (q_lens + extra).tolist()
    q_lens = q_lens.tolist()
    spare = 70
    q = (torch.randn(sum(q_lens) + spare, hq, 128, generator=g) * 0.5).to(torch.bfloat16).to(device)
    k = (torch.randn(sum(k_lens), hkv, 128, generator=g) * 0.5).to(torch.bfloat16).to(device)
    v = (torch.randn(sum(k_lens), hkv, 128, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
    cuq, cuk = offsets(q_lens, device), offsets(k_lens, device)
    out = torch.full_like(q, float("nan"))
    res = flash_attn_varlen_func(q, k, v, cuq, cuk, max(q_lens), max(k_lens), causal=True,
                                 return_softmax_lse=True, out=out)
    lse = res[1]
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True)
    rows = torch.arange(sum(q_lens))
    assert_parity(out[rows], lse[:, rows], ref[rows], ref_lse[:, rows], torch.bfloat16)
    # This build's bar on rows that see at least 32 keys (rows seeing a few
    # keys output near single V rows, where bf16 rounding alone nears 1e-2).
    many, start = [], 0
    for n, m in zip(q_lens, k_lens):
        many += [start + i for i in range(n) if m - n + i + 1 >= 32]
        start += n
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=torch.tensor(many))
    assert torch.isnan(out[sum(q_lens):].float()).all(), "spare rows past the last request were written"


@pytest.mark.parametrize("hkv", [8, 2])
def test_mixed_batch_compact_work_list(device, hkv):
    """Mixed chunked prefill + decode with 8 or 2 KV heads: the compact work
    list gives single-query requests no prefill workgroups."""
    g = torch.Generator().manual_seed(5)
    page, hq, d = 16, 16, 128
    q_lens = [1, 300, 1, 1, 77, 1, 2, 129]
    k_lens = [900, 700, 1, 4000, 77, 33, 2, 1000]
    cols = max((n + page - 1) // page for n in k_lens)
    pool = cols * len(k_lens)
    table = torch.randperm(pool, generator=g).int().reshape(len(k_lens), cols)
    kc = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16).to(device)
    vc = (torch.randn(pool, page, hkv, d, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    cuq = offsets(q_lens, device)
    used = torch.tensor(k_lens, dtype=torch.int32, device=device)
    out, lse = vllm.flash_attn_varlen_func(q, kc, vc, max(q_lens), cuq, cols * page, seqused_k=used,
                                           block_table=table.to(device), causal=True, return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, kc, vc, cuq, used_k=used, block_table=table, causal=True)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    many, start = [], 0
    for n, m in zip(q_lens, k_lens):
        many += [start + i for i in range(n) if m - n + i + 1 >= 32]
        start += n
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=torch.tensor(many))


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_diffkv_192_128_large_grid(device, causal):
    """A DIFFKV launch of more than 2048 workgroups; sampled rows of every
    request against the fp64 oracle."""
    q_lens = [2048, 1500, 3000, 1800]
    hq, hkv = 32, 16
    q, k, v, cuq, cuk = _case_dims(device, torch.bfloat16, 192, 128, hq, hkv, q_lens, q_lens, seed=11 + causal)
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens),
                         max_seqlen_k=max(q_lens), causal=causal)
    g = torch.Generator().manual_seed(3)
    rows = torch.randperm(sum(q_lens), generator=g)[:96].sort().values
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal, rows=rows)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=rows)


@pytest.mark.parametrize("d", [32, 72, 80, 96])
@pytest.mark.parametrize("paged", [False, True])
def test_prefill_padded_dims_ignore_neighbouring_columns(device, d, paged):
    """Head dims 32/72/80/96 run in the 64/128-dim tiles.  K, V and out are
    views into wider NaN-filled storage, so the columns the tile reads or
    computes past d hold NaN: results must still match the oracle, the MFMA
    route must be the one taken, and out's columns past d stay untouched."""
    g = torch.Generator().manual_seed(d + 7 * paged)
    hq, hkv, width, page = 8, 2, 128, 16
    q_lens, k_lens = [5, 130, 257], [40, 130, 300]
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    cuq = offsets(q_lens, device)
    if paged:
        cols = max((n + page - 1) // page for n in k_lens)
        pool = cols * len(k_lens) + 2
        table = torch.randperm(pool, generator=g)[:cols * len(k_lens)].int().reshape(len(k_lens), cols)
        kst = torch.full((pool, page, hkv, width), float("nan"), dtype=torch.bfloat16, device=device)
        vst = torch.full_like(kst, float("nan"))
        k, v = kst[..., :d], vst[..., :d]
        k.copy_((torch.randn(pool, page, hkv, d, generator=g) * 0.5).to(torch.bfloat16))
        v.copy_((torch.randn(pool, page, hkv, d, generator=g) * VALUE_SCALE).to(torch.bfloat16))
        used = torch.tensor(k_lens, dtype=torch.int32, device=device)
        kw = dict(cu_seqlens_k=None, seqused_k=used, block_table=table.to(device))
        ref_kw = dict(used_k=used, block_table=table)
        cuk = None
    else:
        kst = torch.full((sum(k_lens), hkv, width), float("nan"), dtype=torch.bfloat16, device=device)
        vst = torch.full_like(kst, float("nan"))
        k, v = kst[..., :d], vst[..., :d]
        k.copy_((torch.randn(sum(k_lens), hkv, d, generator=g) * 0.5).to(torch.bfloat16))
        v.copy_((torch.randn(sum(k_lens), hkv, d, generator=g) * VALUE_SCALE).to(torch.bfloat16))
        cuk = offsets(k_lens, device)
        kw = dict(cu_seqlens_k=cuk, seqused_k=None, block_table=None)
        ref_kw = dict()
    ost = torch.full((sum(q_lens), hq, width), float("nan"), dtype=torch.bfloat16, device=device)
    out = ost[..., :d]
    lse = torch.empty(hq, q.shape[0], device=device)
    common = dict(max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), softmax_scale=None, causal=True,
                  window_size=(-1, -1), alibi_slopes=None, softcap=0., s_aux=None, q_descale=None,
                  k_descale=None, v_descale=None, mask_mod=None, aux_tensors=None, leftpad_k=None)
    assert _uses_mfma(q, k, v, out, lse, cu_seqlens_q=cuq, **kw, **common)
    res, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=kw["cu_seqlens_k"], seqused_k=kw["seqused_k"],
                         block_table=kw["block_table"], max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
                         causal=True, out=out)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, **ref_kw)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    assert torch.isnan(ost[..., d:].float()).all(), "columns past the head dim were written"


@pytest.mark.parametrize("window", [(0, -1), (1, -1), (31, -1), (64, -1), (100, -1), (700, -1)])
def test_prefill_causal_left_window(device, window):
    """Causal sliding window on the MFMA kernel: row qa sees keys
    [qa - WL, qa]; workgroups skip tiles left of their rows' windows."""
    q_lens, k_lens = [1, 37, 300, 64, 513, 1000], [5, 37, 300, 200, 700, 1000]
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, 8, 2, q_lens, k_lens, scale=0.5, seed=window[0])
    out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens),
                         max_seqlen_k=max(k_lens), causal=True, window_size=window)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, window=window)
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)
    many, start = [], 0
    for n, m in zip(q_lens, k_lens):
        many += [start + i for i in range(n) if min(m - n + i + 1, window[0] + 1) >= 32]
        start += n
    if many:
        assert_parity(out, lse, ref, ref_lse, torch.bfloat16, rows=torch.tensor(many))


@pytest.mark.parametrize("window", [(-1, 0), (-1, 50), (40, 40), (200, -1), (0, 0), (3, 130)])
@pytest.mark.parametrize("paged", [False, True])
def test_prefill_two_sided_window(device, window, paged):
    """Non-causal left/right windows (q_len != k_len, lower-right aligned),
    packed and paged, with GQA and sinks."""
    g = torch.Generator().manual_seed(window[0] * 7 + window[1] + paged)
    hq, hkv, d, page = 8, 2, 64, 16
    q_lens, k_lens = [3, 129, 260, 64], [40, 129, 300, 600]
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
    sinks = torch.randn(hq, generator=g).to(device)
    cuq = offsets(q_lens, device)
    if paged:
        cols = max((n + page - 1) // page for n in k_lens)
        table = torch.randperm(cols * len(k_lens), generator=g).int().reshape(len(k_lens), cols)
        k = (torch.randn(cols * len(k_lens), page, hkv, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
        v = (torch.randn(cols * len(k_lens), page, hkv, d, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
        used = torch.tensor(k_lens, dtype=torch.int32, device=device)
        out, lse = attention(q, k, v, cu_seqlens_q=cuq, seqused_k=used, block_table=table.to(device),
                             max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), window_size=window, s_aux=sinks)
        ref, ref_lse = oracle_attention(q, k, v, cuq, used_k=used, block_table=table, window=window,
                                           sinks=sinks.cpu())
    else:
        k = (torch.randn(sum(k_lens), hkv, d, generator=g) * 0.5).to(torch.bfloat16).to(device)
        v = (torch.randn(sum(k_lens), hkv, d, generator=g) * VALUE_SCALE).to(torch.bfloat16).to(device)
        cuk = offsets(k_lens, device)
        out, lse = attention(q, k, v, cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens),
                             max_seqlen_k=max(k_lens), window_size=window, s_aux=sinks)
        ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, window=window, sinks=sinks.cpu())
    assert_parity(out, lse, ref, ref_lse, torch.bfloat16)


def test_prefill_window_route_is_mfma(device):
    q, k, v, cuq, cuk = _case(device, torch.bfloat16, 128, 16, 8, [300, 17], [300, 17])
    out = torch.empty_like(q)
    lse = torch.empty(16, q.shape[0], device=device)
    assert _uses_mfma(q, k, v, out, lse, cu_seqlens_q=cuq, cu_seqlens_k=cuk, seqused_k=None, max_seqlen_q=300,
                      max_seqlen_k=300, block_table=None, softmax_scale=None, causal=True, window_size=(63, 0),
                      alibi_slopes=None, softcap=0., s_aux=None, q_descale=None, k_descale=None, v_descale=None,
                      mask_mod=None, aux_tensors=None, leftpad_k=None)


@pytest.mark.parametrize("dtype,spread", [(torch.bfloat16, 4.0), (torch.float16, 1.0)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [64, 128])
def test_prefill_negative_scale(device, dtype, spread, causal, d):
    """A negative softmax_scale (the score is scale * q.k for any sign): the
    row max must be that of the scaled scores, and masked keys must stay at
    zero weight (a -inf raw score times a negative scale is +inf).  With x4
    inputs a 64-key tile spans more than 2^128 in probability, so a max taken
    on the raw dot products overflows."""
    q_lens, k_lens = [5, 300, 1000, 64], [5, 300, 1100, 64]
    q, k, v, cuq, cuk = _case(device, dtype, d, 8, 2, q_lens, k_lens, scale=spread, seed=31 + d)
    v = v * 0.5   # peaked rows output single V rows: |out| < 1 keeps one bf16 ulp under the bar
    scale = -d ** -0.5
    kw = dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens),
              causal=causal, softmax_scale=scale)
    out = torch.empty_like(q)
    assert _uses_mfma(q, k, v, out, torch.empty(8, q.shape[0], device=device), **kw)
    out, lse = attention(q, k, v, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=causal, scale=scale)
    assert torch.isfinite(out).all()
    assert_parity(out, lse, ref, ref_lse)


def test_prefill_negative_descale_e4m3_cache(device):
    """E4M3 K/V with a negative k_descale on some (request, KV head) pairs:
    the score scale's sign differs per workgroup."""
    q_lens, k_lens = [40, 700, 129], [40, 900, 129]
    g = torch.Generator().manual_seed(41)
    q = (torch.randn(sum(q_lens), 8, 128, generator=g) * 2.0).to(torch.bfloat16)
    k = (torch.randn(sum(k_lens), 2, 128, generator=g) * 2.0).to(torch.float8_e4m3fn)
    v = (torch.randn(sum(k_lens), 2, 128, generator=g) * 0.5).to(torch.float8_e4m3fn)
    kd = torch.tensor([[1.5, -1.0], [-0.75, 1.0], [-1.25, -0.5]])
    vd = torch.rand(3, 2, generator=g) * 0.5 + 0.5
    cuq, cuk = offsets(q_lens), offsets(k_lens)
    kw = dict(cu_seqlens_q=cuq.to(device), cu_seqlens_k=cuk.to(device), max_seqlen_q=max(q_lens),
              max_seqlen_k=max(k_lens), causal=True, k_descale=kd.to(device), v_descale=vd.to(device))
    qd, kdv, vdv = q.to(device), k.to(device), v.to(device)
    assert _uses_mfma(qd, kdv, vdv, torch.empty_like(qd), torch.empty(8, qd.shape[0], device=device), **kw)
    out, lse = attention(qd, kdv, vdv, **kw)
    ref, ref_lse = oracle_attention(q, k, v, cuq, cuk, causal=True, k_descale=kd, v_descale=vd)
    assert torch.isfinite(out).all()
    assert_parity(out, lse, ref, ref_lse)
