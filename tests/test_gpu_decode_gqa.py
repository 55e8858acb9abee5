"""The matrix-core decode for GQA groups of 3 or more query heads per KV head
(csrc/decode_gqa.h) against the CPU oracle.

It runs for 16-bit queries over K/V of their type or E4M3 (with descales)
at Dqk = Dv in {64, 128}: 32 head
columns per workgroup (groups of 48 and 64 take two), 4 waves each streaming
their own 32-key stages.  The cases cover the stage edges (0, 1, 31, 32, 33
keys and long contexts), split counts, sinks, softcap, left windows, left
padding whose slots hold NaN (rows before a split's first key must never be
read), NaN-poisoned slots past each request, packed and paged K/V (pages of
16 and 48 tokens) and sentinels around a caller-owned output.  Parity bar:
fp16 2e-3, bf16 1e-2, LSE 1e-4 max-abs.

The same kernel takes 2-16 query rows per request (speculative decode) with
any group: 32 (head, row) columns per workgroup, each column with its own
causal/window key range.  64-dim heads stored next to each other run in
pairs when both heads' columns fit one tile (two KV heads as one 128-dim
virtual head, each column keeping its own head's half; E4M3 caches, or 8+
KV heads), also for groups of 1 and 2: paired groups of 1-16 heads, per-head
descales, and heads that do not pair (strided, an odd head count, groups
past 16 heads, 16-bit caches with few KV heads) are covered.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd._decode import decode_rows, gqa_pack, uses_gqa_kernel
from harness import assert_parity, decode_attention, kernel_args, oracle_attention, problem

pytestmark = pytest.mark.gpu


def _i32(values, device):
    return torch.tensor(values, device=device, dtype=torch.int32)


def _pool(stored, page, kv_heads, dim, dtype, device, seed, valid_from):
    """Paged K/V of a permuted pool: slot j of request b is real for
    valid_from[b] <= j < stored[b] and NaN elsewhere (padding and tails)."""
    g = torch.Generator().manual_seed(seed)
    cols = max(-(-n // page) for n in stored) + 1
    pool = len(stored) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(stored), cols)
    kc = torch.randn(pool, page, kv_heads, dim, generator=g)
    vc = torch.randn(pool, page, kv_heads, dim, generator=g) * 0.5
    for b, n in enumerate(stored):
        for pos in list(range(0, valid_from[b])) + list(range(n, cols * page)):
            kc[table[b, pos // page], pos % page] = float("nan")
            vc[table[b, pos // page], pos % page] = float("nan")
    return kc.to(dtype).to(device), vc.to(dtype).to(device), table.to(device), cols


@pytest.mark.parametrize("heads,kv_heads", [(3, 1), (8, 2), (5, 1), (8, 1), (14, 2), (32, 1), (48, 1), (64, 2),
                                             (6, 2), (48, 2), (30, 6), (32, 8), (40, 8), (16, 16), (16, 8)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_groups_dims_and_splits(device, heads, kv_heads, d, dtype, splits):
    lengths, page = [1, 31, 32, 33, 0, 300, 2049, 77], 16
    kc, vc, table, cols = _pool(lengths, page, kv_heads, d, dtype, device, 700 + heads + d + splits,
                                [0] * len(lengths))
    g = torch.Generator().manual_seed(701 + heads + d)
    q = torch.randn(len(lengths), heads, d, generator=g).to(dtype).to(device)
    cu_q, used = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32), _i32(lengths, device)
    sinks = torch.linspace(-2, 2, heads, device=device)
    buffer = torch.full((len(lengths), heads + 8, d), 7.0, device=device, dtype=dtype)
    kw = dict(cu_seqlens_q=cu_q, seqused_k=used, block_table=table, s_aux=sinks)
    p = problem(q, kc, vc, max_seqlen_q=1, max_seqlen_k=cols * page, **kw)
    # Groups of 1 and 2 take this kernel only with paired 64-dim heads.
    assert uses_gqa_kernel(p) == (heads // kv_heads >= 3 or (d == 64 and gqa_pack(p) == 2))
    assert gqa_pack(p) == (2 if d == 64 and (heads, kv_heads) in ((32, 8), (40, 8), (16, 16), (16, 8)) else 1)
    got, lse = decode_attention(q, kc, vc, max_seqlen_k=cols * page, num_splits=splits, out=buffer[:, :heads], **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, sinks=sinks)
    assert_parity(got, lse, ref, ref_lse)
    assert (buffer[:, heads:] == 7.0).all(), "a head slot past the call was stored"


@pytest.mark.parametrize("window", [(-1, -1), (0, 0), (45, 0), (1000, -1)])
@pytest.mark.parametrize("splits", [0, 2])
@pytest.mark.parametrize("page", [16, 48])
@pytest.mark.parametrize("heads,kv_heads,d", [(32, 2, 128), (32, 8, 64)])
def test_softcap_windows_and_left_padding(device, window, splits, page, heads, kv_heads, d):
    """Left padding of 0-17 slots holding NaN before each request's keys; a
    left window then starts a split in the middle of a 16-key group (32 / 8
    heads of 64 dims: paired KV heads)."""
    lengths, left = [1, 40, 777, 0, 1500, 33], [0, 5, 17, 3, 0, 16]
    stored = [n + p for n, p in zip(lengths, left)]
    kc, vc, table, cols = _pool(stored, page, kv_heads, d, torch.bfloat16, device, 710 + page + splits, left)
    g = torch.Generator().manual_seed(711)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cu_q, used, pads = (torch.arange(len(lengths) + 1, device=device, dtype=torch.int32), _i32(lengths, device),
                        _i32(left, device))
    sinks = torch.linspace(-1, 1, heads, device=device)
    kw = dict(cu_seqlens_q=cu_q, seqused_k=used, block_table=table, leftpad_k=pads, window_size=window,
              softcap=30.0, s_aux=sinks)
    keep = []
    probe = kernel_args(q, kc, vc, torch.empty_like(q), torch.empty(heads, len(lengths), device=device), keep=keep,
                        max_seqlen_q=1, max_seqlen_k=cols * page, **kw)
    assert _lib.supported("fa_decode_supported", probe)
    got, lse = decode_attention(q, kc, vc, max_seqlen_k=cols * page, num_splits=splits, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, leftpad=left, window=window,
                                    softcap=30.0, sinks=sinks)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("d", [64, 128])
def test_packed_keys_explicit_scale_and_descales(device, d):
    """Packed K/V rows (cu_seqlens_k), softmax_scale 1/8 and per-(request,
    KV head) descales of a 16-bit cache (they scale the scores and the output)."""
    k_lens, heads, kv_heads = [3, 257, 0, 64, 129], 16, 2
    g = torch.Generator().manual_seed(720 + d)
    q = torch.randn(len(k_lens), heads, d, generator=g).to(torch.float16)
    k = torch.randn(sum(k_lens), kv_heads, d, generator=g).to(torch.float16)
    v = (torch.randn(sum(k_lens), kv_heads, d, generator=g) * 0.5).to(torch.float16)
    kd = torch.rand(len(k_lens), kv_heads, generator=g) * 0.5 + 0.75
    vd = torch.rand(len(k_lens), kv_heads, generator=g) * 0.5 + 0.5
    cu_q = torch.arange(len(k_lens) + 1, dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(k_lens).cumsum(0)), dtype=torch.int32)
    got, lse = decode_attention(q.to(device), k.to(device), v.to(device), cu_seqlens_q=cu_q.to(device),
                                cu_seqlens_k=cu_k.to(device), max_seqlen_k=max(k_lens), softmax_scale=0.125,
                                k_descale=kd.to(device), v_descale=vd.to(device))
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, scale=0.125, k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("heads,kv_heads", [(8, 1), (16, 2), (64, 2), (48, 2), (24, 8), (16, 16), (8, 4)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("splits", [0, 3])
def test_e4m3_caches_with_descales(device, heads, kv_heads, d, q_dtype, splits):
    """E4M3 K/V (widened exactly to the query type in LDS / registers) with
    per-(request, KV head) k/v descales, sinks and softcap 30; NaN-free E4M3
    codes of N(0, 1) values, NaN-poisoned slots past each request."""
    lengths, page = [1, 31, 33, 0, 300, 2049, 77], 16
    g = torch.Generator().manual_seed(730 + heads + d + splits)
    cols = max(-(-n // page) for n in lengths) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols)
    kc = torch.randn(pool, page, kv_heads, d, generator=g).to(torch.float8_e4m3fn)
    vc = torch.randn(pool, page, kv_heads, d, generator=g).to(torch.float8_e4m3fn)
    for b, n in enumerate(lengths):
        for pos in range(n, cols * page):
            kc[table[b, pos // page], pos % page] = float("nan")
            vc[table[b, pos // page], pos % page] = float("nan")
    q = torch.randn(len(lengths), heads, d, generator=g).to(q_dtype)
    kd = torch.rand(len(lengths), kv_heads, generator=g) * 0.1 + 0.05
    vd = torch.rand(len(lengths), kv_heads, generator=g) * 0.25 + 0.25
    sinks = torch.linspace(-2, 2, heads)
    cu_q, used = torch.arange(len(lengths) + 1, dtype=torch.int32), torch.tensor(lengths, dtype=torch.int32)
    kw = dict(cu_seqlens_q=cu_q.to(device), seqused_k=used.to(device), block_table=table.to(device),
              s_aux=sinks.to(device), softcap=30.0, k_descale=kd.to(device), v_descale=vd.to(device))
    p = problem(q.to(device), kc.to(device), vc.to(device), max_seqlen_q=1, max_seqlen_k=cols * page, **kw)
    # Groups of 1-2 take this kernel with paired 64-dim heads only (128-dim
    # E4M3 pairs of such groups run on the VALU decode).
    assert uses_gqa_kernel(p) == (heads // kv_heads >= 3 or (d == 64 and gqa_pack(p) == 2))
    assert gqa_pack(p) == (2 if (heads, kv_heads) in ((16, 2), (24, 8), (16, 16), (8, 4)) else 1)
    got, lse = decode_attention(q.to(device), kc.to(device), vc.to(device), max_seqlen_k=cols * page,
                                num_splits=splits, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, sinks=sinks, softcap=30.0,
                                    k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


def _rows_call(q, kc, vc, q_lens, *, max_seqlen_k, **kw):
    """The multi-row decode (decode_rows) of requests with q_lens query rows;
    fails if the matrix-core kernel does not take the call."""
    device = q.device
    cu_q = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0)), dtype=torch.int32, device=device)
    p = problem(q, kc, vc, cu_seqlens_q=cu_q, max_seqlen_q=max(q_lens), max_seqlen_k=max_seqlen_k, **kw).validate()
    assert uses_gqa_kernel(p)
    out = torch.empty((p.tokens, p.heads, p.dim_v), dtype=p.output_dtype, device=device)
    done = decode_rows(p, out)
    assert done is not None, "the matrix-core decode did not take the call"
    return done, cu_q.cpu()


@pytest.mark.parametrize("q_lens", [[2, 1, 2, 0, 2], [4, 3, 1, 4, 2], [8, 8, 5, 1, 7], [16, 9, 1, 16]])
@pytest.mark.parametrize("heads,kv_heads", [(8, 8), (32, 8), (16, 1), (40, 4)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_rows_per_request(device, q_lens, heads, kv_heads, causal, splits):
    """2-16 query rows per request at the end of each context (speculative
    decode): rows of one request see bottom-right-aligned causal prefixes (or
    every key), requests have fewer rows than max_seqlen_q or none, and
    contexts run 0-2049 keys (a causal row may see no key at all)."""
    d = 128
    lengths = [max(n, 1) + x for n, x in zip(q_lens, [0, 40, 2000, 7, 300, 33])]
    lengths[0] = q_lens[0] - 1 if q_lens[0] > 1 else 0   # fewer keys than rows
    page = 16
    kc, vc, table, cols = _pool(lengths, page, kv_heads, d, torch.bfloat16, device, 740 + heads + splits,
                                [0] * len(lengths))
    g = torch.Generator().manual_seed(741 + sum(q_lens))
    q = torch.randn(sum(q_lens), heads, d, generator=g).to(torch.bfloat16).to(device)
    used = _i32(lengths, device)
    sinks = torch.linspace(-2, 2, heads, device=device)
    kw = dict(seqused_k=used, block_table=table, s_aux=sinks, causal=causal, num_splits=splits)
    (got, lse), cu_q = _rows_call(q, kc, vc, q_lens, max_seqlen_k=cols * page, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, sinks=sinks, causal=causal)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("window", [(0, 0), (45, 0), (20, 3), (1000, -1)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("splits", [0, 2])
@pytest.mark.parametrize("heads,kv_heads", [(16, 4), (32, 8)])
@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.float8_e4m3fn])
def test_rows_windows_softcap_leftpad(device, window, d, splits, heads, kv_heads, kv_dtype):
    """Multi-row decode with left/right windows (each row's own window),
    softcap 30, descales and NaN left padding, over 16-bit and E4M3 caches
    (paired KV heads filling one tile: 32 / 8 heads of 64 dims at 4 rows,
    and every E4M3 case here)."""
    q_lens, left = [3, 4, 1, 4, 2], [0, 5, 17, 3, 16]
    lengths = [3, 40, 777, 1500, 33]
    stored = [n + p for n, p in zip(lengths, left)]
    kc, vc, table, cols = _pool(stored, 48, kv_heads, d, kv_dtype, device, 750 + d + splits, left)
    g = torch.Generator().manual_seed(751 + d)
    q = torch.randn(sum(q_lens), heads, d, generator=g).to(torch.float16).to(device)
    kd = torch.rand(len(q_lens), kv_heads, generator=g) * 0.5 + 0.75
    vd = torch.rand(len(q_lens), kv_heads, generator=g) * 0.5 + 0.5
    used, pads = _i32(lengths, device), _i32(left, device)
    kw = dict(seqused_k=used, block_table=table, leftpad_k=pads, window_size=window, causal=window[1] == 0,
              softcap=30.0, k_descale=kd.to(device), v_descale=vd.to(device), num_splits=splits)
    (got, lse), cu_q = _rows_call(q, kc, vc, q_lens, max_seqlen_k=cols * 48, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, leftpad=left, window=window,
                                    causal=window[1] == 0, softcap=30.0, k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("q_lens", [[2, 2, 1], [5, 8, 3]])
@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,d", [(32, 128), (32, 64), (24, 64)])
def test_rows_e4m3_cache(device, q_lens, q_dtype, heads, d):
    """Multi-row decode over an E4M3 paged cache with descales and sinks
    (64-dim heads in pairs: 24 / 8 heads at 4 rows put 6 heads of two KV
    heads in one tile)."""
    kv_heads, page = 8, 16
    lengths = [300, 2049, 77]
    g = torch.Generator().manual_seed(760 + sum(q_lens))
    cols = max(-(-n // page) for n in lengths) + 1
    table = torch.randperm(len(lengths) * cols, generator=g).int().reshape(len(lengths), cols)
    kc = torch.randn(len(lengths) * cols, page, kv_heads, d, generator=g).to(torch.float8_e4m3fn)
    vc = torch.randn(len(lengths) * cols, page, kv_heads, d, generator=g).to(torch.float8_e4m3fn)
    q = torch.randn(sum(q_lens), heads, d, generator=g).to(q_dtype)
    kd = torch.rand(len(lengths), kv_heads, generator=g) * 0.1 + 0.05
    vd = torch.rand(len(lengths), kv_heads, generator=g) * 0.25 + 0.25
    sinks = torch.linspace(-2, 2, heads)
    used = torch.tensor(lengths, dtype=torch.int32)
    kw = dict(seqused_k=used.to(device), block_table=table.to(device), s_aux=sinks.to(device), causal=True,
              k_descale=kd.to(device), v_descale=vd.to(device))
    (got, lse), cu_q = _rows_call(q.to(device), kc.to(device), vc.to(device), q_lens, max_seqlen_k=cols * page, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, sinks=sinks, causal=True,
                                    k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("layout", ["pairs", "strided", "odd"])
@pytest.mark.parametrize("kind,d", [(torch.bfloat16, 64), (torch.float8_e4m3fn, 64), (torch.float8_e4m3fn, 128)])
def test_head_pairs_and_unpaired_layouts(device, layout, kind, d):
    """64-dim heads and 128-dim E4M3 heads: neighbouring KV heads run in
    pairs; heads of a cache sliced from wider rows (head stride 2 d) and an
    odd KV head count run one KV head per workgroup.  Per-(request, KV head)
    descales differ between the two heads of a pair, so a column scaled with
    its neighbour's descale fails the bar."""
    lengths, page = [1, 31, 33, 0, 300, 2049, 77], 16
    kv_heads = 3 if layout == "odd" else 8
    heads = 6 * kv_heads
    g = torch.Generator().manual_seed(770 + len(layout))
    cols = max(-(-n // page) for n in lengths) + 1
    pool = len(lengths) * cols
    table = torch.randperm(pool, generator=g).int().reshape(len(lengths), cols)
    width = 2 * d if layout == "strided" else d
    kc = torch.randn(pool, page, kv_heads, width, generator=g).to(kind)
    vc = (torch.randn(pool, page, kv_heads, width, generator=g) * 0.5).to(kind)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16)
    kd = torch.rand(len(lengths), kv_heads, generator=g) * 0.5 + 0.5
    vd = torch.rand(len(lengths), kv_heads, generator=g) * 0.5 + 0.5
    if kind == torch.float8_e4m3fn:
        kd, vd = kd * 0.1, vd * 0.5
    cu_q, used = torch.arange(len(lengths) + 1, dtype=torch.int32), torch.tensor(lengths, dtype=torch.int32)
    kg, vg = kc.to(device)[..., :d], vc.to(device)[..., :d]
    kw = dict(cu_seqlens_q=cu_q.to(device), seqused_k=used.to(device), block_table=table.to(device),
              k_descale=kd.to(device), v_descale=vd.to(device))
    p = problem(q.to(device), kg, vg, max_seqlen_q=1, max_seqlen_k=cols * page, **kw)
    assert uses_gqa_kernel(p)
    assert gqa_pack(p) == (2 if layout == "pairs" else 1)
    got, lse = decode_attention(q.to(device), kg, vg, max_seqlen_k=cols * page, **kw)
    ref, ref_lse = oracle_attention(q, kc[..., :d], vc[..., :d], cu_q, used_k=used, block_table=table,
                                    k_descale=kd, v_descale=vd)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (32, 8), (64, 4)])
def test_fp32_output_keeps_fp32_accuracy(device, heads, kv_heads):
    """An fp32 output is held to the fp32 bar (1e-4): such calls skip the
    matrix-core decode, whose P.V rounds probabilities to 16 bits."""
    lengths, page, d = [1, 300, 2049, 0, 77], 16, 128
    kc, vc, table, cols = _pool(lengths, page, kv_heads, d, torch.bfloat16, device, 780 + heads, [0] * len(lengths))
    g = torch.Generator().manual_seed(781)
    q = torch.randn(len(lengths), heads, d, generator=g).to(torch.bfloat16).to(device)
    cu_q, used = torch.arange(len(lengths) + 1, device=device, dtype=torch.int32), _i32(lengths, device)
    out = torch.empty(len(lengths), heads, d, device=device, dtype=torch.float32)
    kw = dict(cu_seqlens_q=cu_q, seqused_k=used, block_table=table)
    assert not uses_gqa_kernel(problem(q, kc, vc, max_seqlen_q=1, max_seqlen_k=cols * page, out=out, **kw))
    got, lse = decode_attention(q, kc, vc, max_seqlen_k=cols * page, out=out, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table)
    assert_parity(got, lse, ref, ref_lse)


def _work_order_lengths(batch, seed):
    """Contexts of 0 keys, exact multiples of the spans the split plan picks
    (no short last split), one key either side of them, and random lengths,
    shuffled over the batch."""
    g = torch.Generator().manual_seed(seed)
    fixed = [0, 1, 127, 128, 129, 256, 384, 512, 513, 1023, 1024, 1025]
    lengths = [fixed[b] if b < len(fixed) else int(torch.randint(0, 700, (1,), generator=g)) for b in range(batch)]
    return [lengths[i] for i in torch.randperm(batch, generator=g).tolist()], g


@pytest.mark.parametrize("batch", [63, 64, 65, 130, 256, 257, 300])
@pytest.mark.parametrize("splits", [0, 1, 4])
def test_work_order_across_request_counts(device, batch, splits):
    """The kernel hands its (split, request) slots out longest first for up
    to 256 requests (64 per pass of a wave) and in grid order past that; with
    full splits, short last splits of every length class, empty requests and
    unused slots in one launch, each request's result must land in its own
    rows (a sentinel-filled output shows any slot stored twice or never)."""
    heads, kv_heads, d, page = 8, 2, 64, 16
    lengths, g = _work_order_lengths(batch, 790 + batch + splits)
    kc, vc, table, cols = _pool(lengths, page, kv_heads, d, torch.bfloat16, device, 791 + batch, [0] * batch)
    q = torch.randn(batch, heads, d, generator=g).to(torch.bfloat16).to(device)
    cu_q, used = torch.arange(batch + 1, device=device, dtype=torch.int32), _i32(lengths, device)
    buffer = torch.full((batch, heads + 4, d), 7.0, device=device, dtype=torch.bfloat16)
    kw = dict(cu_seqlens_q=cu_q, seqused_k=used, block_table=table)
    assert uses_gqa_kernel(problem(q, kc, vc, max_seqlen_q=1, max_seqlen_k=cols * page, **kw))
    got, lse = decode_attention(q, kc, vc, max_seqlen_k=cols * page, num_splits=splits, out=buffer[:, :heads], **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table)
    assert_parity(got, lse, ref, ref_lse)
    assert (buffer[:, heads:] == 7.0).all(), "a head slot past the call was stored"


@pytest.mark.parametrize("batch", [70, 256, 260])
def test_rows_work_order_with_empty_requests(device, batch):
    """Multi-row calls over many requests, some with no query row (no slot
    at all) and some with fewer keys than rows."""
    heads, kv_heads, d, page = 16, 4, 128, 16
    lengths, g = _work_order_lengths(batch, 795 + batch)
    q_lens = torch.randint(0, 5, (batch,), generator=g).tolist()
    q_lens[0] = 4
    kc, vc, table, cols = _pool(lengths, page, kv_heads, d, torch.bfloat16, device, 796 + batch, [0] * batch)
    q = torch.randn(sum(q_lens), heads, d, generator=g).to(torch.bfloat16).to(device)
    used = _i32(lengths, device)
    kw = dict(seqused_k=used, block_table=table, causal=True)
    (got, lse), cu_q = _rows_call(q, kc, vc, q_lens, max_seqlen_k=cols * page, **kw)
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, causal=True)
    assert_parity(got, lse, ref, ref_lse)
