"""Seeded randomized sweep of the decode routes against the oracle.

Each case draws a GQA shape (1-8 KV heads, groups 1-32), head dim 64/128,
bf16/fp16 queries over same-type or E4M3 K/V (with descales), 1-8 query rows
per request (requests with fewer rows than max_seqlen_q, none at all, or
fewer keys than rows), 0-3000 keys in pages of 16/32/48 tokens, causal or
not, left/right windows, softcap, sinks and explicit split counts, then runs
it through the public router (VALU decode, matrix-core decode or prefill,
whichever takes it) at the parity bar: fp16 2e-3, bf16 1e-2, LSE 1e-4.
"""
import random

import pytest
import torch

from harness import assert_parity, attention, offsets, oracle_attention

pytestmark = pytest.mark.gpu


def _draw(seed):
    rng = random.Random(seed)
    kvh = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16, 32])
    rows = rng.choice([1, 1, 1, 2, 3, 4, 8])
    batch = rng.randint(1, 6)
    c = dict(kvh=kvh, hq=kvh * group, d=rng.choice([64, 128, 128]),
             qdt=rng.choice([torch.bfloat16, torch.float16]), fp8=rng.random() < 0.35, rows=rows,
             lengths=[rng.choice([0, 1, 5, 31, 32, 33, 100, 777, 2049, 3000]) for _ in range(batch)],
             page=rng.choice([16, 32, 48]), causal=rng.random() < 0.7,
             window=rng.choice([(-1, -1), (-1, -1), (100, 0), (1000, -1), (40, 3)]),
             cap=rng.choice([0.0, 0.0, 30.0]), sinks=rng.random() < 0.4, splits=rng.choice([0, 0, 1, 3]))
    c["q_lens"] = [1] * batch if rows == 1 else [0 if rng.random() < 0.1 else rng.randint(1, rows) for _ in range(batch)]
    if c["window"][1] == 3:
        c["causal"] = False
    if sum(c["q_lens"]) == 0:
        c["q_lens"][0] = 1
    return c


@pytest.mark.parametrize("seed", range(60))
def test_random_decode_case(device, seed):
    c = _draw(7000 + seed)
    B, kvh, d, page = len(c["lengths"]), c["kvh"], c["d"], c["page"]
    g = torch.Generator().manual_seed(7000 + seed)
    cols = max(-(-max(n, 1) // page) for n in c["lengths"]) + 1
    table = torch.randperm(B * cols, generator=g).int().reshape(B, cols)
    kc = torch.randn(B * cols, page, kvh, d, generator=g)
    vc = torch.randn(B * cols, page, kvh, d, generator=g) * 0.5
    kd = vd = None
    if c["fp8"]:
        kc, vc = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
        kd = torch.rand(B, kvh, generator=g) * 0.5 + 0.25
        vd = torch.rand(B, kvh, generator=g) * 0.5 + 0.25
    else:
        kc, vc = kc.to(c["qdt"]), vc.to(c["qdt"])
    q = torch.randn(sum(c["q_lens"]), c["hq"], d, generator=g).to(c["qdt"])
    sinks = torch.randn(c["hq"], generator=g) if c["sinks"] else None
    cu_q, used = offsets(c["q_lens"]), torch.tensor(c["lengths"], dtype=torch.int32)
    on = lambda t: None if t is None else t.to(device)
    out, lse = attention(q.to(device), kc.to(device), vc.to(device), cu_seqlens_q=cu_q.to(device),
                         seqused_k=used.to(device), block_table=table.to(device),
                         max_seqlen_q=max(c["rows"], max(c["q_lens"])), max_seqlen_k=cols * page,
                         causal=c["causal"], window_size=c["window"], softcap=c["cap"], s_aux=on(sinks),
                         num_splits=c["splits"], k_descale=on(kd), v_descale=on(vd))
    ref, ref_lse = oracle_attention(q, kc, vc, cu_q, used_k=used, block_table=table, causal=c["causal"],
                                    window=c["window"], softcap=c["cap"], sinks=sinks, k_descale=kd, v_descale=vd)
    assert_parity(out, lse, ref, ref_lse, what=str({k: v for k, v in c.items() if k != "qdt"}))
