"""Batch invariance of the fixed-order route (vLLM num_splits=1 /
deterministic) at benchmark config 5's shape.

The reference promises that explicit num_splits=1 selects a batch-invariant
calculation (docs/contracts.md:76-79, tests/test_vllm.py:152-160).  Here a
request's output and LSE must be bit-identical whether it runs alone, in the
full config-5 batch (8 chunks of 512 new tokens on prefixes U[0, 4096] plus
120 single-query requests with contexts U[256, 16384]; DIFFKV Dqk 192 / Dv
128, Hq = Hkv = 16, bf16, 16-token pages, per-head sinks), or in a reordered
sub-batch with other neighbours; and the fixed-order results must still meet
the parity bar against the fp64 oracle.  The chunks take the MFMA prefill
kernel (fa_prefill_supported holds for the deterministic arguments) and the
single-query requests the decode kernel with one split, alone or batched, so
each row is reduced in an order of its own request only.
"""
import pytest
import torch

from flash_attn_mps_amd import _lib, vllm
from harness import assert_parity, kernel_args, offsets, oracle_attention

pytestmark = pytest.mark.gpu

HQ = HKV = 16
DQK, DV, PAGE = 192, 128, 16


@pytest.fixture(scope="module")
def config5():
    device = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(123 + 5)
    prefixes = torch.randint(0, 4097, (8,), generator=g).tolist()
    dec_ctx = torch.randint(256, 16385, (120,), generator=g).tolist()
    q_lens = [512] * 8 + [1] * 120
    k_lens = [p + 512 for p in prefixes] + dec_ctx
    cols = max(-(-n // PAGE) for n in k_lens)
    pool = sum(-(-n // PAGE) for n in k_lens)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(k_lens), cols, dtype=torch.int32)
    start = 0
    for b, n in enumerate(k_lens):
        used = -(-n // PAGE)
        table[b, :used] = perm[start:start + used].int()
        start += used
    gd = torch.Generator(device=device).manual_seed(555)
    kc = torch.randn(pool, PAGE, HKV, DQK, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    vc = (torch.randn(pool, PAGE, HKV, DV, generator=gd, device=device, dtype=torch.float32) * 0.5).to(torch.bfloat16)
    q = (torch.randn(sum(q_lens), HQ, DQK, generator=g) * 0.5).to(torch.bfloat16).to(device)
    sinks = torch.randn(HQ, generator=g).to(device)
    return dict(q_lens=q_lens, k_lens=k_lens, q=q, kc=kc, vc=vc, table=table.to(device), sinks=sinks)


def _call(c, requests, **extra):
    """The vLLM call over the listed requests (in that order)."""
    q_lens = [c["q_lens"][b] for b in requests]
    k_lens = [c["k_lens"][b] for b in requests]
    starts = [sum(c["q_lens"][:b]) for b in requests]
    q = torch.cat([c["q"][s:s + n] for s, n in zip(starts, q_lens)])
    table = c["table"][torch.tensor(requests, device=c["table"].device)]
    used = torch.tensor(k_lens, dtype=torch.int32, device=q.device)
    return vllm.flash_attn_varlen_func(q, c["kc"], c["vc"], max(q_lens), offsets(q_lens, q.device), max(k_lens),
                                       seqused_k=used, block_table=table, causal=True, s_aux=c["sinks"],
                                       return_softmax_lse=True, **extra)


def _rows(c, requests, b):
    """Packed rows of request b inside a call over `requests`."""
    i = requests.index(b)
    start = sum(c["q_lens"][r] for r in requests[:i])
    return slice(start, start + c["q_lens"][b])


def test_fixed_order_route_kernels(config5, device):
    c = config5
    q_lens, k_lens = c["q_lens"], c["k_lens"]
    out = torch.empty(sum(q_lens), HQ, DV, dtype=torch.bfloat16, device=device)
    lse = torch.empty(HQ, sum(q_lens), device=device)
    keep = []
    args = kernel_args(c["q"], c["kc"], c["vc"], out, lse, keep=keep, cu_seqlens_q=offsets(q_lens, device),
                       seqused_k=torch.tensor(k_lens, dtype=torch.int32, device=device), max_seqlen_q=512,
                       max_seqlen_k=max(k_lens), block_table=c["table"], causal=True, s_aux=c["sinks"],
                       deterministic=True, num_splits=1)
    assert _lib.supported("fa_prefill_supported", args)
    args.max_seqlen_q = 1
    assert _lib.supported("fa_decode_supported", args)


def test_requests_are_bit_identical_alone_and_batched(config5):
    c = config5
    everyone = list(range(len(c["q_lens"])))
    full, full_lse = _call(c, everyone, num_splits=1)
    again, again_lse = _call(c, everyone, num_splits=1)
    assert torch.equal(full, again) and torch.equal(full_lse, again_lse)
    longest_decode = max(range(8, 128), key=lambda b: c["k_lens"][b])
    picks = [0, 3, 7, 8, 9, 64, 127, longest_decode]
    for b in picks:
        alone, alone_lse = _call(c, [b], num_splits=1)
        rows = _rows(c, everyone, b)
        assert torch.equal(alone, full[rows]), f"request {b} differs alone vs batched"
        assert torch.equal(alone_lse, full_lse[:, rows]), f"request {b} LSE differs alone vs batched"
    # A reordered sub-batch: decode requests first, then chunks, other neighbours.
    subset = [127, 64, 9, longest_decode, 7, 0, 3] if longest_decode not in (127, 64, 9) else [127, 64, 9, 7, 0, 3]
    part, part_lse = _call(c, subset, deterministic=True)
    for b in subset:
        rows_part, rows_full = _rows(c, subset, b), _rows(c, everyone, b)
        assert torch.equal(part[rows_part], full[rows_full]), f"request {b} differs in the reordered sub-batch"
        assert torch.equal(part_lse[:, rows_part], full_lse[:, rows_full])


def test_fixed_order_results_meet_the_parity_bar(config5):
    """The fixed-order outputs of a chunk and two decode requests against the
    fp64 oracle (bf16 bar 1e-2, LSE 1e-4)."""
    c = config5
    everyone = list(range(len(c["q_lens"])))
    full, full_lse = _call(c, everyone, num_splits=1)
    table_cpu = c["table"].cpu()
    for b in (2, 8, 100):
        n, m = c["q_lens"][b], c["k_lens"][b]
        pages = table_cpu[b, :-(-m // PAGE)].long()
        local = torch.arange(pages.numel(), dtype=torch.int32).reshape(1, -1)
        start = sum(c["q_lens"][:b])
        q = c["q"][start:start + n].cpu()
        ref, ref_lse = oracle_attention(q, c["kc"][pages].cpu(), c["vc"][pages].cpu(),
                                        torch.tensor([0, n], dtype=torch.int32), used_k=torch.tensor([m]),
                                        block_table=local, causal=True, sinks=c["sinks"].cpu(), chunk=128)
        rows = _rows(c, everyone, b)
        assert_parity(full[rows], full_lse[:, rows], ref, ref_lse, torch.bfloat16, what=f"request {b}")
