"""Seeded randomized sweep of the prefill routes against the oracle.

Each case draws 1-5 requests of 1-1100 query rows over as many or more keys,
GQA 1-4 query heads per KV head, head dims 64/128/256 or DIFFKV 192/128,
bf16/fp16, packed or paged (16/64-token pages) K/V, causal or not, left/right
windows, softcap, sinks, a positive or negative softmax scale and, for 16-bit
128-dim heads, E4M3 K/V with descales, then runs it through the public
router (MFMA prefill, mixed batch or generic kernel) at the parity bar on
every row: fp16 2e-3, bf16 1e-2, LSE 1e-4 (-inf where a row sees no key).
V is drawn as 0.5 N(0, 1), as in config 2.
"""
import random

import pytest
import torch

from harness import assert_parity, attention, offsets, oracle_attention

pytestmark = pytest.mark.gpu


def _draw(seed):
    rng = random.Random(seed)
    dims = rng.choice([(64, 64), (128, 128), (128, 128), (256, 256), (192, 128)])
    kvh = rng.choice([1, 2, 4])
    batch = rng.randint(1, 5)
    q_lens = [rng.choice([1, 7, 64, 129, 300, 1100]) for _ in range(batch)]
    extra = [rng.choice([0, 0, 5, 200]) for _ in range(batch)]
    c = dict(dq=dims[0], dv=dims[1], kvh=kvh, hq=kvh * rng.choice([1, 2, 4]), q_lens=q_lens,
             k_lens=[n + e for n, e in zip(q_lens, extra)], dtype=rng.choice([torch.bfloat16, torch.float16]),
             paged=rng.random() < 0.4, page=rng.choice([16, 64]), causal=rng.random() < 0.7,
             window=rng.choice([(-1, -1), (-1, -1), (128, 0), (40, 40)]), cap=rng.choice([0.0, 0.0, 20.0]),
             sinks=rng.random() < 0.3, neg=rng.random() < 0.15,
             fp8=dims == (128, 128) and rng.random() < 0.25)
    if c["window"] == (40, 40):
        c["causal"] = False
    return c



@pytest.mark.parametrize("seed", range(40))
def test_random_prefill_case(device, seed):
    c = _draw(9000 + seed)
    g = torch.Generator().manual_seed(9000 + seed)
    q = torch.randn(sum(c["q_lens"]), c["hq"], c["dq"], generator=g).to(c["dtype"])
    k = torch.randn(sum(c["k_lens"]), c["kvh"], c["dq"], generator=g)
    v = torch.randn(sum(c["k_lens"]), c["kvh"], c["dv"], generator=g) * 0.5
    kd = vd = None
    if c["fp8"]:
        k, v = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
        kd = torch.rand(len(c["q_lens"]), c["kvh"], generator=g) * 0.5 + 0.5
        vd = torch.rand(len(c["q_lens"]), c["kvh"], generator=g) * 0.5 + 0.5
    else:
        k, v = k.to(c["dtype"]), v.to(c["dtype"])
    cu_q, cu_k = offsets(c["q_lens"]), offsets(c["k_lens"])
    kw, table = {}, None
    if c["paged"]:
        page = c["page"]
        cols = max(-(-n // page) for n in c["k_lens"])
        pool = len(c["k_lens"]) * cols
        table = torch.randperm(pool, generator=g).int().reshape(len(c["k_lens"]), cols)
        kc = torch.zeros(pool, page, c["kvh"], c["dq"], dtype=k.dtype)
        vc = torch.zeros(pool, page, c["kvh"], c["dv"], dtype=v.dtype)
        for b, n in enumerate(c["k_lens"]):
            pos = torch.arange(n)
            src = cu_k[b] + pos
            kc[table[b, pos // page].long(), pos % page] = k[src]
            vc[table[b, pos // page].long(), pos % page] = v[src]
        k, v = kc, vc
        used = torch.tensor(c["k_lens"], dtype=torch.int32)
        kw = dict(seqused_k=used.to(device), block_table=table.to(device))
        okw = dict(used_k=used, block_table=table)
    else:
        kw = dict(cu_seqlens_k=cu_k.to(device))
        okw = dict(cu_k=cu_k)
    scale = (-1.0 if c["neg"] else 1.0) * c["dq"] ** -0.5
    sinks = torch.randn(c["hq"], generator=g) if c["sinks"] else None
    on = lambda t: None if t is None else t.to(device)
    out, lse = attention(q.to(device), k.to(device), v.to(device), cu_seqlens_q=cu_q.to(device),
                         max_seqlen_q=max(c["q_lens"]), max_seqlen_k=max(c["k_lens"]), causal=c["causal"],
                         window_size=c["window"], softcap=c["cap"], s_aux=on(sinks), softmax_scale=scale,
                         k_descale=on(kd), v_descale=on(vd), **kw)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, causal=c["causal"], window=c["window"], softcap=c["cap"],
                                    sinks=sinks, scale=scale, k_descale=kd, v_descale=vd, chunk=512, **okw)
    what = str({key: val for key, val in c.items() if key != "dtype"})
    assert_parity(out, lse, ref, ref_lse, what=what)
