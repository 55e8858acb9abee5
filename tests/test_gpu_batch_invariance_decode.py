"""Batch invariance of the fixed-order route (vLLM num_splits=1) where the
single-query rows take the decode kernels: config 3's shape (Llama-3-8B:
32 query / 8 KV heads, d128, 16-token pages, contexts past 4096 keys) on the
matrix-core GQA decode, with a bf16 and an E4M3 cache, and config 4's shape
(Gemma-2-9B: 16 / 8 heads, d256, E4M3 cache with [B, Hkv] descales, softcap
50, window (4095, 0)).

The reference promises that num_splits=1 selects a batch-invariant
calculation (docs/contracts.md:76-79, tests/test_vllm.py:152-159).  Each
request's output and LSE must be bit-identical when it runs alone, with all
the single-query requests, and next to a multi-row chunk (the mixed-batch
route: the chunk on the MFMA prefill, the single-query rows on the decode
kernel with one split).  The three calls reach the decode kernel through
different argument builders (decode() for single-query calls, the mixed
batch's copy of the prefill arguments); the results must not depend on it.
The fixed-order results also meet the parity bar against the fp64 oracle.
"""
import pytest
import torch

from flash_attn_mps_amd import vllm
from harness import assert_parity, offsets, oracle_attention

pytestmark = pytest.mark.gpu

PAGE = 16
E4M3 = torch.float8_e4m3fn


def _cache(device, k_lens, hkv, d, seed, fp8):
    """Paged K/V (a shuffled pool of 16-token pages); E4M3 caches hold codes
    of N(0,1) / descale, descales U[0.01, 0.1] per KV head."""
    g = torch.Generator().manual_seed(seed)
    n_pages = [-(-n // PAGE) for n in k_lens]
    pool = sum(n_pages)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(k_lens), max(n_pages), dtype=torch.int32)
    at = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[at:at + n].int()
        at += n
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    k = torch.randn(pool, PAGE, hkv, d, generator=gd, device=device)
    v = torch.randn(pool, PAGE, hkv, d, generator=gd, device=device)
    desc = None
    if fp8:
        desc = torch.empty(len(k_lens), hkv).uniform_(0.01, 0.1, generator=g).to(device)
        # One descale per KV head for the whole pool (each request's pages
        # are its own, so per-request descales would need a per-page map):
        # the test uses request 0's row for every request.
        desc = desc[:1].expand(len(k_lens), hkv).contiguous()
        # Saturating at +-448 as store_kvcache does (torch's cast maps
        # out-of-range values to NaN codes).
        k = (k / desc[0][None, None, :, None]).clamp(-448, 448).to(E4M3)
        v = (v / desc[0][None, None, :, None]).clamp(-448, 448).to(E4M3)
    else:
        k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    return k, v, table.to(device), desc


def _shape(name, device):
    if name.startswith("config3"):
        fp8 = name.endswith("fp8")
        hq, hkv, d = 32, 8, 128
        k_lens = [600, 3000, 4097, 9000, 20000, 32768, 1234, 5000, 2300]
        q_lens = [1, 1, 1, 1, 1, 1, 1, 1, 300]
        extra = dict(causal=True)
        oracle_extra = dict(causal=True)
    else:
        fp8 = True
        hq, hkv, d = 16, 8, 256
        k_lens = [1024, 4096, 4097, 8192, 6000, 1500, 2500]
        q_lens = [1, 1, 1, 1, 1, 1, 200]
        extra = dict(causal=True, softcap=50.0, window_size=(4095, 0))
        oracle_extra = dict(causal=True, softcap=50.0, window=(4095, 0))
    k, v, table, desc = _cache(device, k_lens, hkv, d, seed=len(name), fp8=fp8)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(sum(q_lens), hq, d, generator=g).to(torch.bfloat16).to(device)
    if desc is not None:
        extra = dict(extra, k_descale=desc, v_descale=desc)
        oracle_extra = dict(oracle_extra, k_descale=desc, v_descale=desc)
    return dict(q=q, k=k, v=v, table=table, q_lens=q_lens, k_lens=k_lens, extra=extra, oracle=oracle_extra,
                hq=hq, d=d)


@pytest.fixture(scope="module", params=["config3 bf16", "config3 fp8", "config4 fp8"])
def case(request):
    return _shape(request.param, torch.device("cuda", 0))


def _call(c, requests):
    q_lens = [c["q_lens"][b] for b in requests]
    k_lens = [c["k_lens"][b] for b in requests]
    starts = [sum(c["q_lens"][:b]) for b in requests]
    q = torch.cat([c["q"][s:s + n] for s, n in zip(starts, q_lens)])
    idx = torch.tensor(requests, device=q.device)
    extra = dict(c["extra"])
    for name in ("k_descale", "v_descale"):
        if name in extra:
            extra[name] = extra[name][idx]
    return vllm.flash_attn_varlen_func(q, c["k"], c["v"], max(q_lens), offsets(q_lens, q.device), max(k_lens),
                                       seqused_k=torch.tensor(k_lens, dtype=torch.int32, device=q.device),
                                       block_table=c["table"][idx], num_splits=1, return_softmax_lse=True, **extra)


def _rows(c, requests, b):
    i = requests.index(b)
    start = sum(c["q_lens"][r] for r in requests[:i])
    return slice(start, start + c["q_lens"][b])


def test_single_query_rows_alone_together_and_next_to_a_chunk(case):
    c = case
    singles = [b for b, n in enumerate(c["q_lens"]) if n == 1]
    everyone = list(range(len(c["q_lens"])))
    together, together_lse = _call(c, singles)
    mixed, mixed_lse = _call(c, everyone)
    again, again_lse = _call(c, everyone)
    assert torch.equal(mixed, again) and torch.equal(mixed_lse, again_lse)
    for b in singles:
        alone, alone_lse = _call(c, [b])
        rt, rm = _rows(c, singles, b), _rows(c, everyone, b)
        assert torch.equal(alone, together[rt]), f"request {b}: alone vs all single-query requests"
        assert torch.equal(alone_lse, together_lse[:, rt]), f"request {b}: LSE alone vs together"
        assert torch.equal(alone, mixed[rm]), f"request {b}: alone vs next to a multi-row chunk"
        assert torch.equal(alone_lse, mixed_lse[:, rm]), f"request {b}: LSE alone vs mixed"
    # A reordered sub-batch with the chunk first.
    chunk = [b for b, n in enumerate(c["q_lens"]) if n > 1]
    subset = chunk + singles[::-2]
    part, part_lse = _call(c, subset)
    for b in subset:
        rp, rm = _rows(c, subset, b), _rows(c, everyone, b)
        assert torch.equal(part[rp], mixed[rm]), f"request {b}: reordered sub-batch"
        assert torch.equal(part_lse[:, rp], mixed_lse[:, rm])


def test_fixed_order_results_meet_the_parity_bar(case):
    c = case
    everyone = list(range(len(c["q_lens"])))
    mixed, mixed_lse = _call(c, everyone)
    table = c["table"].cpu()
    for b in (0, 5, len(everyone) - 1):
        n, m = c["q_lens"][b], c["k_lens"][b]
        pages = table[b, :-(-m // PAGE)].long()
        local = torch.arange(pages.numel(), dtype=torch.int32).reshape(1, -1)
        start = sum(c["q_lens"][:b])
        okw = dict(c["oracle"])
        for name in ("k_descale", "v_descale"):
            if name in okw:
                okw[name] = okw[name][b:b + 1].cpu()
        ref, ref_lse = oracle_attention(c["q"][start:start + n].cpu(), c["k"][pages.to(c["k"].device)].cpu(),
                                        c["v"][pages.to(c["v"].device)].cpu(),
                                        torch.tensor([0, n], dtype=torch.int32), used_k=torch.tensor([m]),
                                        block_table=local, chunk=128, **okw)
        rows = _rows(c, everyone, b)
        assert_parity(mixed[rows], mixed_lse[:, rows], ref, ref_lse, torch.bfloat16, what=f"request {b}")
