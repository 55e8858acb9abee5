"""Public FlashAttention-2 API on gfx950 against the CPU oracle.

The request shapes, lengths and edge cases are data from the reference's
own suite (flash_attn_mps tests/test_interface.py, cited per case); the
checks are this build's: parity at the north-star bar (bf16 1e-2, fp16 2e-3,
fp32 1e-4, LSE 1e-4 max-abs), exact cache bytes, untouched sentinels, and
outputs bit-identical across equivalent entry points.
"""
import pytest
import torch

import flash_attn_mps_amd as fa
from harness import assert_parity, offsets, oracle_attention, seeded

pytestmark = pytest.mark.gpu


def _flat_lse(lse):
    """Dense LSE [B, Hq, S] -> the oracle's [Hq, B*S]."""
    return lse.transpose(0, 1).flatten(1)


# Ragged requests with GQA 4/2: a one-row request, a request with fewer keys
# than queries... (test_interface.py:11-25: cu_q [0,1,4,21], cu_k [0,5,8,25]).
RAGGED_Q, RAGGED_K = (1, 3, 17), (5, 3, 17)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dqk,dv", [(40, 40), (128, 128), (192, 128), (256, 256), (512, 512)])
def test_varlen_ragged_causal_gqa(device, dtype, dqk, dv):
    seed = 1000 + dqk + dv
    q = seeded((sum(RAGGED_Q), 4, dqk), seed, dtype, device)
    k = seeded((sum(RAGGED_K), 2, dqk), seed + 1, dtype, device)
    v = seeded((sum(RAGGED_K), 2, dv), seed + 2, dtype, device, scale=0.5)
    cu_q, cu_k = offsets(RAGGED_Q, device), offsets(RAGGED_K, device)
    out, lse = fa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 17, 17, causal=True, return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, causal=True)
    assert out.shape == (21, 4, dv) and lse.shape == (4, 21)
    assert_parity(out, lse, ref, ref_lse)


# Dense batches whose query and key lengths differ, and an empty query
# length (test_interface.py:28-38).
@pytest.mark.parametrize("sq,sk", [(2, 5), (5, 2), (0, 3), (37, 129)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dense_lower_right_alignment(device, sq, sk, dtype):
    q = seeded((2, sq, 4, 32), 11, dtype, device)
    k = seeded((2, sk, 2, 32), 12, dtype, device)
    v = seeded((2, sk, 2, 32), 13, dtype, device, scale=0.5)
    out, lse = fa.flash_attn_func(q, k, v, causal=True, return_softmax_lse=True)
    assert out.shape == (2, sq, 4, 32) and lse.shape == (2, 4, sq)
    ref, ref_lse = oracle_attention(q.flatten(0, 1), k.flatten(0, 1), v.flatten(0, 1),
                                    offsets([sq, sq]), offsets([sk, sk]), causal=True)
    assert_parity(out.flatten(0, 1), _flat_lse(lse), ref, ref_lse)


def test_dense_offsets_cache_follows_shape_changes(device):
    """Alternating dense shapes reuse resident offsets without mixing them up
    (shape sequence of test_interface.py:41-53)."""
    for step, (batch, sq, sk) in enumerate(((2, 3, 5), (1, 7, 4), (2, 3, 5), (3, 1, 17), (1, 7, 4))):
        q = seeded((batch, sq, 4, 32), 20 + step, torch.float16, device)
        k = seeded((batch, sk, 2, 32), 40 + step, torch.float16, device)
        v = seeded((batch, sk, 2, 32), 60 + step, torch.float16, device)
        out = fa.flash_attn_func(q, k, v, causal=True)
        ref, _ = oracle_attention(q.flatten(0, 1), k.flatten(0, 1), v.flatten(0, 1),
                                  offsets([sq] * batch), offsets([sk] * batch), causal=True)
        assert_parity(out.flatten(0, 1), None, ref, None, what=f"shape {batch}x{sq}x{sk}")


def test_packed_layouts_match_the_dense_call_bit_for_bit(device):
    """qkv / kv packing are views of the same data, so results are identical
    (layouts of test_interface.py:79-88)."""
    qkv = seeded((2, 7, 3, 4, 32), 77, torch.float16, device)
    q, k, v = qkv.unbind(2)
    expected = fa.flash_attn_func(q, k, v, causal=True)
    cu = offsets([7, 7], device)
    results = {
        "qkvpacked": fa.flash_attn_qkvpacked_func(qkv, causal=True),
        "kvpacked": fa.flash_attn_kvpacked_func(q, qkv[:, :, 1:], causal=True),
        "varlen qkvpacked": fa.flash_attn_varlen_qkvpacked_func(qkv.flatten(0, 1), cu, 7, causal=True),
        "varlen kvpacked": fa.flash_attn_varlen_kvpacked_func(q.flatten(0, 1), qkv.flatten(0, 1)[:, 1:], cu, cu,
                                                              7, 7, causal=True),
    }
    for name, got in results.items():
        assert torch.equal(got.reshape(expected.shape), expected), name


def test_dense_fp8_from_transposed_views(device):
    """E4M3 Q/K/V given as non-contiguous [B, S, H, D] views (transposes of
    [B, H, S, D] storage, as in test_interface.py:91-101); output is fp16."""
    qs = seeded((2, 4, 9, 32), 5, torch.float8_e4m3fn, "cpu")
    ks = seeded((2, 2, 13, 32), 6, torch.float8_e4m3fn, "cpu")
    vs = seeded((2, 2, 13, 32), 7, torch.float8_e4m3fn, "cpu")
    q, k, v = (t.to(device).transpose(1, 2) for t in (qs, ks, vs))
    assert not q.is_contiguous()
    out, lse = fa.flash_attn_func(q, k, v, causal=True, return_softmax_lse=True)
    assert out.dtype == torch.float16
    ref, ref_lse = oracle_attention(*(t.transpose(1, 2).flatten(0, 1) for t in (qs, ks, vs)),
                                    offsets([9, 9]), offsets([13, 13]), causal=True)
    assert_parity(out.flatten(0, 1), _flat_lse(lse), ref, ref_lse)


def test_varlen_paged_views_of_shared_storage(device):
    """K and V are two halves of one [pages, heads, P, 128] parent, read
    through a block table whose unused tail entry is -1
    (test_interface.py:104-113)."""
    parent = seeded((3, 9, 2, 32, 128), 8, torch.float16, device)
    k, v = parent[1].transpose(1, 2).split(64, -1)
    q = seeded((11, 4, 64), 9, torch.float16, device)
    cu_q = torch.tensor([0, 1, 11], device=device, dtype=torch.int32)
    cu_k = torch.tensor([0, 65, 114], device=device, dtype=torch.int32)
    table = torch.tensor([[4, 1, 7], [2, 6, -1]], device=device, dtype=torch.int32)
    before = parent.clone()
    out, lse = fa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 10, 65, causal=True, block_table=table,
                                         return_softmax_lse=True)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, used_k=cu_k.diff(), block_table=table, causal=True)
    assert_parity(out, lse, ref, ref_lse)
    assert torch.equal(parent, before)


def test_kvcache_append_with_batch_index_and_leftpad(device):
    """Append two tokens to dense cache rows chosen by cache_batch_idx, with
    left padding hidden from attention; lengths stay untouched
    (test_interface.py:116-138: rows [3, 1], lengths [9, 11], pads [3, 5])."""
    kc = seeded((4, 23, 2, 32), 30, torch.float16, device)
    vc = seeded((4, 23, 2, 32), 31, torch.float16, device)
    expect_k, expect_v = kc.clone(), vc.clone()
    q = seeded((2, 2, 4, 32), 32, torch.float16, device)
    k = seeded((2, 2, 2, 32), 33, torch.float16, device)
    v = seeded((2, 2, 2, 32), 34, torch.float16, device)
    lengths = torch.tensor([9, 11], device=device, dtype=torch.int32)
    pads = torch.tensor([3, 5], device=device, dtype=torch.int32)
    rows = torch.tensor([3, 1], device=device, dtype=torch.int32)
    out, lse = fa.flash_attn_with_kvcache(q, kc, vc, k, v, cache_seqlens=lengths, cache_batch_idx=rows,
                                          cache_leftpad=pads, causal=True, return_softmax_lse=True)
    for b, (row, end) in enumerate(((3, 9), (1, 11))):
        expect_k[row, end:end + 2], expect_v[row, end:end + 2] = k[b], v[b]
    assert torch.equal(kc, expect_k) and torch.equal(vc, expect_v)
    assert lengths.tolist() == [9, 11]
    ref, ref_lse = oracle_attention(q.flatten(0, 1), kc, vc, offsets([2, 2]), used_k=lengths + 2 - pads,
                                    block_table=rows[:, None], causal=True, leftpad=pads.cpu())
    assert_parity(out.flatten(0, 1), _flat_lse(lse), ref, ref_lse)


def _rotate_pairs(x, cos, sin, interleaved):
    """Rotary embedding of x [..., S, H, D] with cos/sin [S, half] (fp64 on the CPU)."""
    x = x.double().cpu()
    c, s = cos.double().cpu()[:, None, :], sin.double().cpu()[:, None, :]
    half = cos.shape[-1]
    y = x.clone()
    if interleaved:
        a, b = x[..., 0:2 * half:2], x[..., 1:2 * half:2]
        y[..., 0:2 * half:2], y[..., 1:2 * half:2] = a * c - b * s, a * s + b * c
    else:
        a, b = x[..., :half], x[..., half:2 * half]
        y[..., :half], y[..., half:2 * half] = a * c - b * s, a * s + b * c
    return y


@pytest.mark.parametrize("interleaved", [True, False])
def test_kvcache_rotary_then_append(device, interleaved):
    """New q/k rotated at positions 5 and 6 (old length 5) before the append;
    rotary dim 16 of 32 (test_interface.py:141-169)."""
    q = seeded((1, 2, 4, 32), 50, torch.float16, device)
    k = seeded((1, 2, 2, 32), 51, torch.float16, device)
    v = seeded((1, 2, 2, 32), 52, torch.float16, device)
    kc = seeded((1, 16, 2, 32), 53, torch.float16, device)
    vc = seeded((1, 16, 2, 32), 54, torch.float16, device)
    theta = seeded((16, 8), 55, torch.float32, device)
    cos, sin = theta.cos().half(), theta.sin().half()
    lengths = torch.tensor([5], device=device, dtype=torch.int32)
    out, lse = fa.flash_attn_with_kvcache(q, kc, vc, k, v, cos, sin, lengths, causal=True,
                                          rotary_interleaved=interleaved, return_softmax_lse=True)
    k_rot = _rotate_pairs(k[0], cos[5:7], sin[5:7], interleaved)
    assert (kc[0, 5:7].double().cpu() - k_rot).abs().max() <= 2e-3     # one fp16 rounding
    assert torch.equal(vc[0, 5:7], v[0])
    q_rot = _rotate_pairs(q[0], cos[5:7], sin[5:7], interleaved).half()
    ref, ref_lse = oracle_attention(q_rot, kc, vc, offsets([2]), used_k=lengths + 2,
                                    block_table=torch.zeros(1, 1, dtype=torch.int32), causal=True)
    assert_parity(out.flatten(0, 1), _flat_lse(lse), ref, ref_lse)


@pytest.mark.parametrize("old_len", [15, 16, 17, 31, 32])
def test_paged_append_across_page_boundaries(device, old_len):
    """One-token decode steps that append at the end, start or middle of a
    16-token page (test_interface.py:172-187; table [[5, 1, 7]])."""
    kc = seeded((8, 16, 2, 32), 60, torch.float16, device)
    vc = seeded((8, 16, 2, 32), 61, torch.float16, device)
    table = torch.tensor([[5, 1, 7]], device=device, dtype=torch.int32)
    q = seeded((1, 1, 4, 32), 62 + old_len, torch.float16, device)
    k = seeded((1, 1, 2, 32), 63 + old_len, torch.float16, device)
    v = seeded((1, 1, 2, 32), 64 + old_len, torch.float16, device)
    lengths = torch.tensor([old_len], device=device, dtype=torch.int32)
    out, lse = fa.flash_attn_with_kvcache(q, kc, vc, k, v, cache_seqlens=lengths, block_table=table,
                                          causal=True, return_softmax_lse=True)
    page = int(table[0, old_len // 16])
    assert torch.equal(kc[page, old_len % 16], k[0, 0]) and torch.equal(vc[page, old_len % 16], v[0, 0])
    ref, ref_lse = oracle_attention(q.flatten(0, 1), kc, vc, offsets([1]), used_k=lengths + 1,
                                    block_table=table, causal=True)
    assert_parity(out.flatten(0, 1), _flat_lse(lse), ref, ref_lse)


def test_public_checks_run_before_any_launch(device, monkeypatch):
    """Malformed vLLM decode calls raise on the host; the library is never
    called (the argument changes of test_interface.py:56-76)."""
    from flash_attn_mps_amd import _lib
    from flash_attn_mps_amd.vllm import flash_attn_varlen_func

    calls = []
    monkeypatch.setattr(_lib, "call", lambda *a, **k: calls.append(a))
    q = seeded((1, 4, 32), 70, torch.float16, device)
    k = seeded((17, 2, 32), 71, torch.float16, device)
    cu_q = torch.tensor([0, 1], device=device, dtype=torch.int32)
    cu_k = torch.tensor([0, 17], device=device, dtype=torch.int32)
    good = dict(q=q, k=k, v=k, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=1, max_seqlen_k=17)
    bad = {
        "integer queries": dict(q=q.int()),
        "int64 offsets": dict(cu_seqlens_q=cu_q.long()),
        "q/k head dims differ": dict(k=k[..., :16]),
        "integer out": dict(out=torch.empty(1, 4, 32, dtype=torch.int32, device=device)),
        "descale of the wrong shape": dict(k_descale=torch.ones(1, 1, device=device)),
        "sinks for 2 of 4 heads": dict(s_aux=torch.ones(2, device=device)),
        "window bound below -1": dict(window_size=(-2, 0)),
        "two rows for one single-query request": dict(q=q.expand(2, -1, -1)),
        "offsets on the CPU": dict(cu_seqlens_k=cu_k.cpu()),
    }
    for name, change in bad.items():
        with pytest.raises((ValueError, TypeError)):
            flash_attn_varlen_func(**{**good, **change})
        assert not calls, f"{name} reached the library"
