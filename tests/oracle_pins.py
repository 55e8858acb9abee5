"""Checks that pin the CPU attention oracle (oracle/attention.py) to facts
that do not depend on its own formula.

Each check takes an attention function with the oracle's signature and raises
AssertionError when it disagrees with:
* torch.nn.functional.scaled_dot_product_attention (an independent library
  routine) on inputs whose features it can express (GQA by explicit head
  repetition, lower-right causality and windows as torch.tril/triu band
  masks, ALiBi as an additive float mask);
* closed forms: zero queries average V and give LSE = ln L, a single visible
  key returns its V row with LSE = its score, a (0, 0) window returns the
  diagonal row, two-key softcap weights from math.tanh;
* identities between features: sink = rescale by sigmoid(lse - sink) and
  LSE = logaddexp(lse, sink); q/k descales = scaled softmax_scale; v descale
  = scaled output; paged storage through a permuted block table = packed
  storage; leftpad = sliced keys; causal_by_batch = per-request calls; mask
  kinds 1 and 2 reduce to windows at their extreme parameters;
* the reference's golden values (tests/test_attention_core.py:52-63 of
  flash_attn_mps: empty KV with sinks -> out 0, LSE = sink).

tests/test_oracle_mutants.py plants mistakes in copies of the oracle and
shows that every planted mistake fails at least one check.
"""
import math

import torch
import torch.nn.functional as F

F64 = torch.float64


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _cu(lengths):
    c = [0]
    for n in lengths:
        c.append(c[-1] + n)
    return torch.tensor(c, dtype=torch.int32)


def _close(a, b, atol=1e-10, rtol=1e-10, what=""):
    a, b = a.double(), b.double()
    ok = torch.isclose(a, b, atol=atol, rtol=rtol, equal_nan=True) | ((a == b) & torch.isinf(b))
    if not bool(ok.all()):
        err = (a - b).abs()[~ok]
        raise AssertionError(f"{what}: {int((~ok).sum())} mismatches, max diff {float(err.max()):.3e}")


def _sdpa(q, k, v, mask, scale):
    """q [n, H, D], k/v [L, H, D] (heads already repeated) -> [n, H, Dv]."""
    o = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                       attn_mask=mask, scale=scale)
    return o.transpose(0, 1)


def _band(n, length, lo=None, hi=None):
    """Boolean [n, L] mask of keys j with (L - n + i) - lo <= j <= (L - n + i) + hi;
    None leaves that side open.  Built with tril/triu diagonals."""
    m = torch.ones(n, length, dtype=torch.bool)
    if hi is not None:
        m = m.tril(length - n + hi)
    if lo is not None:
        m = m.triu(length - n - lo)
    return m


def _rand(seed, *shape, scale=1.0):
    return torch.randn(*shape, generator=_g(seed), dtype=F64) * scale


# ----------------------------------------------------------------- checks

def check_sdpa_varlen_gqa(attn):
    """Varlen packed requests, GQA 4:2, causal and not, q_len <= k_len."""
    q_lens, k_lens = [5, 9, 1], [5, 13, 7]
    hq, hkv, d, dv = 4, 2, 16, 12
    q = _rand(1, sum(q_lens), hq, d)
    k = _rand(2, sum(k_lens), hkv, d)
    v = _rand(3, sum(k_lens), hkv, dv)
    cuq, cuk = _cu(q_lens), _cu(k_lens)
    for causal in (False, True):
        out, _ = attn(q, k, v, cuq, cuk, causal=causal, scale=0.3)
        for b, (n, length) in enumerate(zip(q_lens, k_lens)):
            qs = q[cuq[b]:cuq[b + 1]]
            ks = k[cuk[b]:cuk[b + 1]].repeat_interleave(hq // hkv, dim=1)
            vs = v[cuk[b]:cuk[b + 1]].repeat_interleave(hq // hkv, dim=1)
            mask = _band(n, length, hi=0) if causal else None
            _close(out[cuq[b]:cuq[b + 1]], _sdpa(qs, ks, vs, mask, 0.3), what=f"sdpa causal={causal} b={b}")


def check_default_scale_diffkv(attn):
    """Default softmax scale is Dqk^-1/2, also when Dv differs."""
    q, k, v = _rand(4, 6, 2, 24), _rand(5, 6, 2, 24), _rand(6, 6, 2, 8)
    cu = _cu([6])
    out, _ = attn(q, k, v, cu, cu)
    _close(out, _sdpa(q, k, v, None, 24 ** -0.5), what="default scale")


def check_zero_query_closed_form(attn):
    """q = 0: every score is 0, so out = mean of visible V rows and LSE = ln(#visible)."""
    q_lens, k_lens = [4, 3], [6, 3]
    q = torch.zeros(sum(q_lens), 2, 8, dtype=F64)
    k, v = _rand(7, sum(k_lens), 2, 8), _rand(8, sum(k_lens), 2, 8)
    out, lse = attn(q, k, v, _cu(q_lens), _cu(k_lens), causal=True)
    row = 0
    for b, (n, length) in enumerate(zip(q_lens, k_lens)):
        base = sum(k_lens[:b])
        for i in range(n):
            seen = length - n + i + 1
            _close(out[row], v[base:base + seen].mean(0), what="zero-q out")
            _close(lse[:, row], torch.full((2,), math.log(seen), dtype=F64), what="zero-q lse")
            row += 1


def check_single_key_closed_form(attn):
    """A row that sees exactly one key returns that V row; LSE = scale * q.k."""
    q, k, v = _rand(9, 3, 1, 8), _rand(10, 5, 1, 8), _rand(11, 5, 1, 6)
    # q_len 3, k_len 5, window (0, 0): row i sees only key 2 + i
    out, lse = attn(q, k, v, _cu([3]), _cu([5]), window=(0, 0), scale=0.7)
    for i in range(3):
        _close(out[i, 0], v[2 + i, 0], what="window(0,0) out")
        _close(lse[0, i], 0.7 * (q[i, 0] @ k[2 + i, 0]), what="window(0,0) lse")
    # causal with more queries than keys: the first rows see nothing -> 0 / -inf
    out, lse = attn(q, k[:1], v[:1], _cu([3]), _cu([1]), causal=True, scale=0.7)
    _close(out[:2], torch.zeros(2, 1, 6, dtype=F64), what="no-key rows out")
    assert bool(torch.isneginf(lse[0, :2]).all()), "no-key rows lse must be -inf"
    _close(out[2, 0], v[0, 0], what="last row sees key 0")


def check_windows_sdpa(attn):
    """Left/right windows and causal+window as tril/triu band masks."""
    q, k, v = _rand(12, 7, 2, 8), _rand(13, 11, 2, 8), _rand(14, 11, 2, 8)
    cuq, cuk = _cu([7]), _cu([11])
    for causal, window in ((False, (2, 1)), (True, (3, -1)), (False, (-1, 0)), (False, (0, 4)),
                           (True, (20, -1))):
        out, _ = attn(q, k, v, cuq, cuk, causal=causal, window=window, scale=0.5)
        lo = window[0] if window[0] >= 0 else None
        hi = 0 if causal else (window[1] if window[1] >= 0 else None)
        if causal and window[1] >= 0:
            hi = min(0, window[1])
        mask = _band(7, 11, lo=lo, hi=hi)
        _close(out, _sdpa(q, k, v, mask, 0.5), what=f"window {window} causal={causal}")


def check_softcap_closed_form(attn):
    """Two keys: weights follow cap * tanh(scale * q.k / cap); a huge cap is no cap."""
    q, k, v = _rand(15, 1, 1, 4, scale=3), _rand(16, 2, 1, 4, scale=3), _rand(17, 2, 1, 3)
    cu1, cu2 = _cu([1]), _cu([2])
    for cap in (0.5, 3.0):
        s = [cap * math.tanh(0.9 * float(q[0, 0] @ k[j, 0]) / cap) for j in range(2)]
        w1 = 1.0 / (1.0 + math.exp(s[0] - s[1]))
        expect = (1 - w1) * v[0, 0] + w1 * v[1, 0]
        out, lse = attn(q, k, v, cu1, cu2, scale=0.9, softcap=cap)
        _close(out[0, 0], expect, atol=1e-12, what=f"softcap {cap} out")
        _close(lse[0, 0], torch.tensor(math.log(math.exp(s[0]) + math.exp(s[1])), dtype=F64), what="softcap lse")
    big, _ = attn(q, k, v, cu1, cu2, scale=0.9, softcap=1e12)
    plain, _ = attn(q, k, v, cu1, cu2, scale=0.9)
    _close(big, plain, atol=1e-9, what="softcap -> inf")


def check_alibi_sdpa(attn):
    """ALiBi = additive float mask -slope * |qpos - kpos| ([Hq] and [B, Hq] slopes)."""
    q_lens, k_lens = [4, 6], [9, 6]
    q, k, v = _rand(18, 10, 2, 8), _rand(19, 15, 2, 8), _rand(20, 15, 2, 8)
    slopes = torch.tensor([[0.5, 0.125], [0.25, 1.0]], dtype=F64)
    for per_batch in (False, True):
        al = slopes if per_batch else slopes[0]
        out, _ = attn(q, k, v, _cu(q_lens), _cu(k_lens), causal=True, alibi=al, scale=0.4)
        for b, (n, length) in enumerate(zip(q_lens, k_lens)):
            s = slopes[b] if per_batch else slopes[0]
            qpos = torch.arange(length - n, length, dtype=F64)[:, None]
            kpos = torch.arange(length, dtype=F64)[None, :]
            bias = -s[:, None, None] * (qpos - kpos).abs()
            bias = bias.masked_fill(~_band(n, length, hi=0), -math.inf)
            ref = _sdpa(q[sum(q_lens[:b]):sum(q_lens[:b + 1])], k[sum(k_lens[:b]):sum(k_lens[:b + 1])],
                        v[sum(k_lens[:b]):sum(k_lens[:b + 1])], bias, 0.4)
            _close(out[sum(q_lens[:b]):sum(q_lens[:b + 1])], ref, what=f"alibi per_batch={per_batch}")


def check_sink_identity(attn):
    """A sink s rescales out by sigmoid(lse - s) and gives LSE = logaddexp(lse, s)."""
    q, k, v = _rand(21, 5, 3, 8), _rand(22, 5, 3, 8), _rand(23, 5, 3, 8)
    cu = _cu([5])
    sinks = torch.tensor([-2.0, 0.5, 4.0], dtype=F64)
    base, lse = attn(q, k, v, cu, cu, causal=True)
    out, lse_s = attn(q, k, v, cu, cu, causal=True, sinks=sinks)
    factor = torch.sigmoid(lse - sinks[:, None]).transpose(0, 1).unsqueeze(-1)
    _close(out, base * factor, what="sink out")
    _close(lse_s, torch.logaddexp(lse, sinks[:, None].expand_as(lse)), what="sink lse")


def check_empty_kv_golden(attn):
    """flash_attn_mps tests/test_attention_core.py:52-63: empty KV -> out 0,
    LSE -inf, or LSE = sink with sinks [-10, 0, 1, 10]."""
    q = _rand(24, 13, 4, 32)
    k = torch.empty(0, 2, 32, dtype=F64)
    cuq, cuk = torch.tensor([0, 7, 13], dtype=torch.int32), torch.tensor([0, 0, 0], dtype=torch.int32)
    out, lse = attn(q, k, k, cuq, cuk)
    assert int(torch.count_nonzero(out)) == 0 and bool(torch.isneginf(lse).all()), "empty KV"
    sinks = torch.tensor([-10.0, 0.0, 1.0, 10.0], dtype=F64)
    out, lse = attn(q, k, k, cuq, cuk, sinks=sinks)
    assert int(torch.count_nonzero(out)) == 0, "empty KV with sinks: out"
    _close(lse, sinks[:, None].expand(4, 13), what="empty KV with sinks: lse")


def check_descale_identities(attn):
    """q/k descales multiply the score; v descale multiplies the output ([B, Hkv] per request)."""
    q_lens = [3, 4]
    q, k, v = _rand(25, 7, 4, 8), _rand(26, 7, 2, 8), _rand(27, 7, 2, 8)
    cu = _cu(q_lens)
    qd = torch.tensor([[0.5, 2.0], [1.5, 0.25]], dtype=F64)
    kd = torch.tensor([[3.0, 0.5], [0.75, 2.0]], dtype=F64)
    vd = torch.tensor([[2.0, 0.125], [4.0, 0.5]], dtype=F64)
    out, lse = attn(q, k, v, cu, cu, causal=True, q_descale=qd, k_descale=kd, v_descale=vd, scale=0.3)
    for b in range(2):
        rows = slice(sum(q_lens[:b]), sum(q_lens[:b + 1]))
        for h in range(4):
            g = h // 2
            o1, l1 = attn(q[rows, h:h + 1], k[rows, g:g + 1], v[rows, g:g + 1], _cu([q_lens[b]]),
                          _cu([q_lens[b]]), causal=True, scale=0.3 * float(qd[b, g] * kd[b, g]))
            _close(out[rows, h], o1[:, 0] * vd[b, g], what="descale out")
            _close(lse[h, rows], l1[0], what="descale lse")


def check_paged_equals_packed(attn):
    """Paged K/V read through a permuted block table (and leftpad) equals the
    packed request keys."""
    page, lengths, left = 4, [7, 10], [1, 0]
    q = _rand(28, 2 + 5, 2, 8)
    q_lens = [2, 5]
    pages_per = 4
    table = torch.tensor([[5, 2, 7, 0], [1, 6, 3, 4]], dtype=torch.int32)
    kc, vc = _rand(29, 8, page, 1, 8), _rand(30, 8, page, 1, 6)
    out, lse = attn(q, kc, vc, _cu(q_lens), used_k=torch.tensor(lengths), block_table=table, causal=True,
                    leftpad=torch.tensor(left))
    for b in range(2):
        flat_k = kc[table[b].long()].reshape(pages_per * page, 1, 8)
        flat_v = vc[table[b].long()].reshape(pages_per * page, 1, 6)
        ks, vs = flat_k[left[b]:left[b] + lengths[b]], flat_v[left[b]:left[b] + lengths[b]]
        rows = slice(sum(q_lens[:b]), sum(q_lens[:b + 1]))
        o1, l1 = attn(q[rows], ks, vs, _cu([q_lens[b]]), _cu([lengths[b]]), causal=True)
        _close(out[rows], o1, what="paged out")
        _close(lse[:, rows], l1, what="paged lse")


def check_packed_leftpad_and_used(attn):
    """Packed keys start at cu_k[b] + leftpad[b]; seqused_k limits the count."""
    q, k, v = _rand(31, 3, 1, 8), _rand(32, 12, 1, 8), _rand(33, 12, 1, 8)
    out, _ = attn(q, k, v, _cu([3]), _cu([12]), used_k=torch.tensor([5]), leftpad=torch.tensor([4]),
                  causal=True)
    o1, _ = attn(q, k[4:9], v[4:9], _cu([3]), _cu([5]), causal=True)
    _close(out, o1, what="leftpad packed")


def check_causal_by_batch(attn):
    q_lens, k_lens = [3, 4], [5, 4]
    q, k, v = _rand(34, 7, 2, 8), _rand(35, 9, 2, 8), _rand(36, 9, 2, 8)
    flags = torch.tensor([True, False])
    out, _ = attn(q, k, v, _cu(q_lens), _cu(k_lens), causal=flags)
    for b in range(2):
        rows = slice(sum(q_lens[:b]), sum(q_lens[:b + 1]))
        keys = slice(sum(k_lens[:b]), sum(k_lens[:b + 1]))
        o1, _ = attn(q[rows], k[keys], v[keys], _cu([q_lens[b]]), _cu([k_lens[b]]), causal=bool(flags[b]))
        _close(out[rows], o1, what="causal_by_batch")


class _Mask:
    def __init__(self, kind, width=-1, clamp=False):
        self.kind, self.sliding_window_left, self.clamp_prefix_to_window = kind, width, clamp


def check_mask_kinds_reduce_to_windows(attn):
    """Kind 2 (rswa) with prefix 0 = causal window (width - 1); prefix >= L =
    causal.  Kind 1 (mm_prefix) with no range = causal window (width - 1); a
    range covering every key = full attention, or with clamp = window
    (width - 1, open right).  A range [lo, hi] adds exactly those keys."""
    n, length, w = 6, 9, 3
    q, k, v = _rand(37, n, 2, 8), _rand(38, length, 2, 8), _rand(39, length, 2, 8)
    cuq, cuk = _cu([n]), _cu([length])

    def run(**kw):
        return attn(q, k, v, cuq, cuk, scale=0.5, **kw)[0]

    win, _ = attn(q, k, v, cuq, cuk, scale=0.5, causal=True, window=(w - 1, -1))
    causal, _ = attn(q, k, v, cuq, cuk, scale=0.5, causal=True)
    full, _ = attn(q, k, v, cuq, cuk, scale=0.5)
    left_open, _ = attn(q, k, v, cuq, cuk, scale=0.5, window=(w - 1, -1))
    _close(run(mask=_Mask(2), aux=(torch.tensor([0], dtype=torch.int32), torch.tensor([w]))), win,
           what="kind2 prefix 0")
    _close(run(mask=_Mask(2), aux=(torch.tensor([length]), torch.tensor([w]))), causal, what="kind2 prefix L")
    none = torch.full((n, 2), -1, dtype=torch.int32)
    _close(run(mask=_Mask(1, w), aux=(none,)), win, what="kind1 no range")
    every = torch.tensor([[0, length - 1]] * n, dtype=torch.int32)
    _close(run(mask=_Mask(1, w), aux=(every,)), full, what="kind1 full range")
    _close(run(mask=_Mask(1, w, clamp=True), aux=(every,)), left_open, what="kind1 clamp")
    # rswa with prefix p: keys < p are visible to every row at or after them
    p = 4
    qpos = torch.arange(length - n, length)[:, None]
    kpos = torch.arange(length)[None, :]
    keep = (qpos - kpos >= 0) & ((kpos < p) | (qpos - kpos < w))
    _close(run(mask=_Mask(2), aux=(torch.tensor([p]), torch.tensor([w]))),
           _sdpa(q, k, v, keep, 0.5), what="kind2 prefix p")
    # mm_prefix range [1, 7] on row 0 only
    ranges = none.clone()
    ranges[0] = torch.tensor([1, 7])
    keep = (qpos - kpos >= 0) & (qpos - kpos < w)
    keep[0, 1:8] = True
    _close(run(mask=_Mask(1, w), aux=(ranges,)), _sdpa(q, k, v, keep, 0.5), what="kind1 one range")


def check_rows_subset(attn):
    q_lens = [5, 7]
    q, k, v = _rand(40, 12, 2, 8), _rand(41, 12, 2, 8), _rand(42, 12, 2, 8)
    cu = _cu(q_lens)
    full, lse = attn(q, k, v, cu, cu, causal=True)
    rows = torch.tensor([0, 4, 6, 11])
    part, lse_p = attn(q, k, v, cu, cu, causal=True, rows=rows)
    _close(part[rows], full[rows], what="rows out")
    _close(lse_p[:, rows], lse[:, rows], what="rows lse")


def check_fp8_inputs_dequantize(attn):
    """FP8 K/V holding every finite E4M3 code (flash_attn_mps
    tests/test_attention_core.py:81-98) equal float64 inputs with the decoded
    values."""
    codes = torch.arange(256, dtype=torch.int32)
    codes = codes[(codes != 127) & (codes != 255)].to(torch.uint8)
    raw = codes.repeat(3)[:2 * 16 * 2 * 8].reshape(2 * 16, 2, 8)
    k8 = raw.view(torch.float8_e4m3fn)
    v8 = raw.flip(0).contiguous().view(torch.float8_e4m3fn)
    q = _rand(43, 2, 4, 8, scale=0.01)
    cuq, cuk = _cu([1, 1]), _cu([20, 12])
    out8, lse8 = attn(q, k8, v8, cuq, cuk)
    from oracle import fp8 as ofp8
    kd = torch.from_numpy(ofp8.decode(raw.numpy())).double()
    vd = torch.from_numpy(ofp8.decode(raw.flip(0).contiguous().numpy())).double()
    out, lse = attn(q, kd, vd, cuq, cuk)
    _close(out8, out, what="fp8 out")
    _close(lse8, lse, what="fp8 lse")


ALL_CHECKS = [
    check_sdpa_varlen_gqa, check_default_scale_diffkv, check_zero_query_closed_form,
    check_single_key_closed_form, check_windows_sdpa, check_softcap_closed_form, check_alibi_sdpa,
    check_sink_identity, check_empty_kv_golden, check_descale_identities, check_paged_equals_packed,
    check_packed_leftpad_and_used, check_causal_by_batch, check_mask_kinds_reduce_to_windows,
    check_rows_subset, check_fp8_inputs_dequantize,
]
