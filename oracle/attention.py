"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference attention math.

Follows the semantics of SuperMarioYL/flash-attn-mps tests/reference.py:6-90
(the reference's own fp64 oracle) and of the storage addressing in
flash_attn_mps/kernels/attention.metal:18-51:

* per request b, keys 0..L-1 where L = seqused_k[b] or cu_k[b+1]-cu_k[b]
  (reference.py:19-23);
* paged keys are read at storage position leftpad[b] + j through
  block_table[b, pos // P] (reference.py:43-48, attention.metal:18-27); packed
  keys at row cu_k[b] + leftpad[b] + j (attention.metal:79-82, 124);
* GQA: query head h reads KV head h // (Hq // Hkv) (reference.py:28);
* q/k/v descales multiply q, k and v per (b, kv head) (reference.py:33-53);
* score = scale * q.k, then softcap * tanh(score / softcap), then minus
  slope * |qpos - kpos| (reference.py:54-62, attention.metal:47-51);
* lower-right positions: query row i sits at L - Lq + i (reference.py:57);
* causal keeps kpos <= qpos, windows keep qpos - WL <= kpos <= qpos + WR
  (reference.py:63-68); mask kind 1 / kind 2 replace that rule
  (reference.py:69-80, attention.metal:29-45);
* the sink is an extra logit in the denominator only (reference.py:82-87);
* fully masked rows give output 0 and LSE -inf (reference.py:86-88).

The result is computed in float64 by default (``dtype`` selects float32 for
the CPU throughput baseline).  ``rows`` restricts the computation to a subset
of packed query rows so that full-size configurations can be spot-checked.
"""
import torch


def _to_cpu(x, dtype):
    # float8_e4m3fn widens exactly on the CPU.
    return x.detach().cpu().to(dtype)


def _as_list(t):
    return None if t is None else [int(v) for v in t.detach().cpu().tolist()]


def attention(q, k, v, cu_q, cu_k=None, used_k=None, block_table=None, scale=None,
              causal=False, window=(-1, -1), softcap=0.0, alibi=None, sinks=None,
              q_descale=None, k_descale=None, v_descale=None, mask=None, aux=None,
              leftpad=None, dtype=torch.float64, rows=None):
    """Return (out [T, Hq, Dv], lse [Hq, T]) on the CPU in ``dtype``.

    Rows outside every request, or not listed in ``rows``, are 0 / -inf.
    """
    q, k, v = (_to_cpu(t, dtype) for t in (q, k, v))
    cuq = _as_list(cu_q)
    cuk = _as_list(cu_k)
    lengths = _as_list(used_k) if used_k is not None else [b - a for a, b in zip(cuk, cuk[1:])]
    table = None if block_table is None else block_table.detach().cpu().long()
    left = [0] * len(lengths) if leftpad is None else _as_list(torch.as_tensor(leftpad))
    causal_by_batch = _as_list(causal) if torch.is_tensor(causal) else None
    total, heads, dq = q.shape
    hkv, dv = k.shape[-2], v.shape[-1]
    group = heads // hkv
    kv_of_head = torch.arange(heads) // group
    scale = dq ** -0.5 if scale is None else float(scale)
    out = torch.zeros(total, heads, dv, dtype=dtype)
    lse = torch.full((heads, total), -torch.inf, dtype=dtype)
    selected = None
    if rows is not None:
        selected = torch.zeros(total, dtype=torch.bool)
        selected[torch.as_tensor(rows, dtype=torch.long)] = True

    def per_head(t, b):
        if t is None:
            return None
        return t.detach().cpu().to(dtype)[b][kv_of_head]          # [Hq]

    for b, length in enumerate(lengths):
        start, end = cuq[b], cuq[b + 1]
        if start == end:
            continue
        qlen = end - start
        idx = torch.arange(qlen)
        if selected is not None:
            idx = idx[selected[start:end]]
            if idx.numel() == 0:
                continue
        if table is not None:
            pos = left[b] + torch.arange(length)
            page = k.shape[1]
            phys = table[b, pos // page]
            key, value = k[phys, pos % page], v[phys, pos % page]
        else:
            base = (cuk[b] if cuk is not None else 0) + left[b]
            key, value = k[base:base + length], v[base:base + length]
        key = key[:, kv_of_head].transpose(0, 1)                     # [Hq, L, Dqk]
        value = value[:, kv_of_head].transpose(0, 1)                 # [Hq, L, Dv]
        query = q[start + idx].transpose(0, 1)                       # [Hq, n, Dqk]
        for name, t, target in (("q", q_descale, "query"), ("k", k_descale, "key"),
                                ("v", v_descale, "value")):
            s = per_head(t, b)
            if s is None:
                continue
            if target == "query":
                query = query * s[:, None, None]
            elif target == "key":
                key = key * s[:, None, None]
            else:
                value = value * s[:, None, None]
        scores = torch.matmul(query, key.transpose(-2, -1)) * scale   # [Hq, n, L]
        if softcap:
            scores = torch.tanh(scores / softcap) * softcap
        qpos = (length - qlen + idx)[:, None]                         # [n, 1]
        kpos = torch.arange(length)[None, :]                          # [1, L]
        diff = qpos - kpos
        if alibi is not None:
            slopes = alibi.detach().cpu().to(dtype)
            slopes = slopes if slopes.ndim == 1 else slopes[b]
            scores = scores - slopes[:, None, None] * diff.abs().to(dtype)
        is_causal = causal_by_batch[b] if causal_by_batch is not None else bool(causal)
        kind = getattr(mask, "kind", 0) if mask is not None else 0
        if kind == 1:
            width = mask.sliding_window_left
            ranges = aux[0].detach().cpu().long()[start + idx]       # [n, 2]
            keep = diff >= 0
            if width >= 0:
                keep &= diff < width
            lo, hi = ranges[:, :1], ranges[:, 1:2]
            modality = (lo >= 0) & (kpos >= lo) & (kpos <= hi)
            if mask.clamp_prefix_to_window and width >= 0:
                modality &= diff < width
            keep |= modality
        elif kind == 2:
            prefix_len = int(aux[0].detach().cpu()[b])
            width = int(aux[1].detach().cpu()[0])
            keep = (diff >= 0) & ((kpos < prefix_len) | (diff < width))
        else:
            keep = (diff >= 0) if is_causal else torch.ones(idx.numel(), length, dtype=torch.bool)
            if window[0] >= 0:
                keep = keep & (diff <= window[0])
            if window[1] >= 0:
                keep = keep & (-diff <= window[1])
        scores = scores.masked_fill(~keep, -torch.inf)
        logits = scores
        if sinks is not None:
            sink = sinks.detach().cpu().to(dtype).reshape(heads, 1, 1).expand(-1, idx.numel(), 1)
            logits = torch.cat((scores, sink), dim=-1)
        row_lse = torch.logsumexp(logits, dim=-1)                    # [Hq, n]
        probs = torch.exp(scores - row_lse.unsqueeze(-1)).nan_to_num(0.0)
        out[start + idx] = torch.matmul(probs, value).transpose(0, 1)
        lse[:, start + idx] = row_lse
    return out, lse


def flops(q_lens, k_lens, heads, dqk, dv, causal=True, window_left=-1):
    """Algorithmic FLOPs: visible (query, key) pairs x Hq x 2(Dqk + Dv), lower-right causal."""
    pairs = 0
    for lq, lk in zip(q_lens, k_lens):
        for i in range(lq):
            qpos = lk - lq + i
            hi = min(lk - 1, qpos) if causal else lk - 1
            lo = max(0, qpos - window_left) if window_left >= 0 else 0
            pairs += max(0, hi - lo + 1)
    return pairs * heads * 2 * (dqk + dv)
