"""Attention features through the router, mostly on the generic kernel
(odd head dims, strides, leftpad, empty KV, windows with sinks, FP8 codes,
softcap), against the CPU oracle at the parity bar (fp16 2e-3, bf16 1e-2,
fp32 1e-4, LSE 1e-4).

Shapes, lengths, tables and feature values are data from flash_attn_mps
tests/test_attention_core.py, cited per case.
"""
import pytest
import torch

from harness import assert_parity, attention, max_err, oracle_attention, seeded

pytestmark = pytest.mark.gpu


def _i32(values, device):
    return torch.tensor(values, device=device, dtype=torch.int32)


@pytest.mark.parametrize("dqk,dv", [(1, 1), (7, 19), (57, 99), (255, 129), (257, 33), (1, 511)])
def test_odd_head_dims_with_strided_views(device, dqk, dv):
    """Every tensor a stride-2 view; output into a sentinel buffer; an empty
    first request (test_attention_core.py:10-30)."""
    q = seeded((15, 4, 2 * dqk), 400, torch.float32, device)[2:13, :, ::2]
    k = seeded((19, 2, 2 * dqk), 401, torch.float32, device)[1:18, :, ::2]
    v = seeded((19, 2, 2 * dv), 402, torch.float32, device)[1:18, :, ::2]
    cu_q, cu_k = _i32([0, 0, 4, 11], device), _i32([0, 3, 8, 17], device)
    buffer = torch.full((15, 4, 2 * dv), 123.0, device=device)
    out = buffer[2:13, :, ::2]
    got, lse = attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=7, max_seqlen_k=9,
                         causal=True, out=out)
    assert got.data_ptr() == out.data_ptr()
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, causal=True)
    assert_parity(got, lse, ref, ref_lse)
    untouched = torch.ones_like(buffer, dtype=torch.bool)
    untouched[2:13, :, ::2] = False
    assert (buffer[untouched] == 123).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_paged_lengths_from_offsets_with_leftpad(device, dtype, splits):
    """Paged keys whose lengths come from cu_seqlens_k (physical pages must
    not add the previous requests' offsets), left padding 5/9/1, K and V
    split from one 160-wide buffer (test_attention_core.py:33-50)."""
    parent = seeded((12, 2, 32, 160), 410, dtype, device)
    k, v = parent.transpose(1, 2).split((96, 64), dim=-1)
    q = seeded((39, 4, 96), 411, dtype, device)
    table = _i32([[7, 2, 9, 1], [4, 6, 3, 10], [5, 8, 0, 11]], device)
    cu_q, cu_k = _i32([0, 1, 6, 39], device), _i32([0, 69, 150, 183], device)
    left = _i32([5, 9, 1], device)
    got, lse = attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=33, max_seqlen_k=81,
                         block_table=table, leftpad_k=left, causal=True, num_splits=splits)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, used_k=cu_k.diff(), block_table=table, leftpad=left.cpu(),
                                    causal=True)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("with_sinks", [False, True])
def test_requests_without_keys(device, with_sinks):
    """No keys at all: output 0, LSE -inf, or the sink logit itself when
    sinks are given, whatever the split count (test_attention_core.py:53-63)."""
    q = seeded((13, 4, 32), 420, torch.float16, device)
    k = torch.empty(0, 2, 32, device=device, dtype=torch.float16)
    sinks = torch.tensor([-10.0, 0.0, 1.0, 10.0], device=device) if with_sinks else None
    out, lse = attention(q, k, k, cu_seqlens_q=_i32([0, 7, 13], device), cu_seqlens_k=_i32([0, 0, 0], device),
                         max_seqlen_q=7, max_seqlen_k=0, s_aux=sinks, num_splits=4)
    assert torch.count_nonzero(out) == 0
    expected = sinks[:, None].expand(4, 13) if with_sinks else torch.full((4, 13), float("-inf"), device=device)
    assert max_err(lse, expected) <= 1e-5


@pytest.mark.parametrize("q_len,k_len", [(257, 1025), (1, 4097)])
def test_peaked_softmax_over_long_keys(device, q_len, k_len):
    """Scores with std ~9 (q and k scaled by 3) over up to 4097 keys
    (test_attention_core.py:66-78).  The 257-row case runs on the MFMA
    kernel, which rounds the weights to fp16 before P.V (error up to about
    2^-10 max|v| on rows dominated by two keys), so values are 0.5*N(0,1)
    as in benchmark config 2."""
    q = seeded((q_len, 4, 128), 430, torch.float16, device, scale=3.0)
    k = seeded((k_len, 2, 128), 431, torch.float16, device, scale=3.0)
    v = seeded((k_len, 2, 128), 432, torch.float16, device, scale=0.5)
    cu_q, cu_k = _i32([0, q_len], device), _i32([0, k_len], device)
    got, lse = attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=q_len, max_seqlen_k=k_len,
                         causal=True)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, causal=True)
    assert_parity(got, lse, ref, ref_lse)


def _all_finite_e4m3(count):
    """The 254 finite E4M3FN codes (every byte but 0x7F / 0xFF), repeated to `count`."""
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes != 0x7F) & (codes != 0xFF)]
    return codes.repeat(-(-count // codes.numel()))[:count].view(torch.float8_e4m3fn)


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16])
def test_every_fp8_code_as_keys_and_values(device, q_dtype):
    """Every finite E4M3 code (subnormals, +-448) appears as a key and as a
    value of a paged decode with descales 1/8 and 1/16
    (test_attention_core.py:81-98)."""
    n = 8 * 16 * 2 * 32
    k = _all_finite_e4m3(n).reshape(8, 16, 2, 32).to(device)
    v = _all_finite_e4m3(n).view(torch.uint8).flip(0).view(torch.float8_e4m3fn).reshape(8, 16, 2, 32).to(device)
    q = seeded((2, 4, 32), 440, q_dtype, device, scale=0.01)
    used = _i32([97, 63], device)
    table = _i32([[5, 0, 7, 2, 6, 4, 1], [2, 1, 4, 3, 0, 0, 0]], device)
    scale = torch.tensor([[0.125, 0.0625]], device=device).expand(2, 2)
    got, lse = attention(q, k, v, cu_seqlens_q=_i32([0, 1, 2], device), seqused_k=used, max_seqlen_q=1,
                         max_seqlen_k=97, block_table=table, k_descale=scale, v_descale=scale)
    ref, ref_lse = oracle_attention(q, k, v, _i32([0, 1, 2], "cpu"), used_k=used, block_table=table,
                                    k_descale=scale, v_descale=scale)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("window,causal", [((0, 0), True), ((15, 2), False), ((-1, 7), False), ((127, -1), True)])
def test_windows_with_sinks_and_empty_splits(device, window, causal):
    """Windows that leave whole splits empty, a request with no keys, sinks
    (test_attention_core.py:101-113: 3 / 35 / 33 queries over 300 / 0 / 7 keys)."""
    q = seeded((71, 4, 32), 450, torch.float16, device)
    k = seeded((307, 2, 32), 451, torch.float16, device)
    v = seeded((307, 2, 32), 452, torch.float16, device)
    cu_q, cu_k = _i32([0, 3, 38, 71], device), _i32([0, 300, 300, 307], device)
    sinks = torch.tensor([-2.0, 0.0, 1.0, 3.0], device=device)
    got, lse = attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=35, max_seqlen_k=300,
                         window_size=window, causal=causal, s_aux=sinks, num_splits=3)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, window=window, causal=causal, sinks=sinks)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("length,width", [(513, 15), (769, 63), (1025, 127)])
def test_local_windows_across_key_lengths(device, length, width):
    """Causal local attention of 3 queries with widths 15 / 63 / 127 over 513
    to 1025 keys, Dv != Dqk (test_attention_core.py:116-131)."""
    q = seeded((3, 4, 64), 460, torch.float16, device)
    k = seeded((length, 2, 64), 461, torch.float16, device)
    v = seeded((length, 2, 32), 462, torch.float16, device)
    cu_q, cu_k = _i32([0, 3], device), _i32([0, length], device)
    got, lse = attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=3, max_seqlen_k=length,
                         window_size=(width, 0), causal=True)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, window=(width, 0), causal=True)
    assert_parity(got, lse, ref, ref_lse)


@pytest.mark.parametrize("dtype,dim", [(torch.float16, 128), (torch.bfloat16, 64), (torch.float32, 256)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("cap", [0.25, 1.0, 3.0])
def test_softcap_with_empty_and_short_requests(device, dtype, dim, causal, cap):
    """Softcaps 0.25 / 1 / 3 (1 is a real cap, not a switch) over a request
    with no keys and two short ones; q and k scaled by 3
    (test_attention_core.py:134-148)."""
    q = seeded((73, 4, dim), 470, dtype, device, scale=3.0)
    k = seeded((100, 2, dim), 471, dtype, device, scale=3.0)
    v = seeded((100, 2, dim), 472, dtype, device, scale=0.5)
    cu_q, cu_k = _i32([0, 3, 38, 73], device), _i32([0, 0, 97, 100], device)
    got, lse = attention(q, k, v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=35, max_seqlen_k=97,
                         causal=causal, softcap=cap)
    ref, ref_lse = oracle_attention(q, k, v, cu_q, cu_k, causal=causal, softcap=cap)
    assert_parity(got, lse, ref, ref_lse)
