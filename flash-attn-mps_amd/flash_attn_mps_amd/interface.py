"""FlashAttention-2 inference API for PyTorch-ROCm tensors on MI355X.

Drop-in for flash_attn_mps/interface.py: the same public functions,
positional order, defaults, keyword-only markers, tensor layouts and LSE
shapes (``[Hq, T]`` for varlen, ``[B, Hq, Sq]`` for dense and KV-cache calls),
on 'cuda' (HIP) tensors where the reference takes 'mps' ones.

Each function only adapts its layout: dense batches become packed rows on
uniform offsets, a dense KV cache becomes a one-column table of cache rows,
packed QKV/KV tensors become views.  The adapted call is a
:class:`~flash_attn_mps_amd._problem.Problem`, validated in full on the host
and then solved by the gfx950 kernels (``_attention.solve``).
"""
from collections import OrderedDict

import torch

from ._attention import solve
from ._problem import MaskSpec, Problem, reject_training  # noqa: F401  (MaskSpec: vLLM masks)

PAGE_MULTIPLE = 16   # paged caches: page sizes the FlashAttention contract accepts


class _UniformOffsets:
    """int32 offsets 0, L, 2L, ..., B*L on a device, made once per (device, B, L).

    Dense layers of one model reuse a handful of shapes, so a small LRU keeps
    their offsets resident and a call adds no host-to-device copy (which also
    keeps dense calls capturable in HIP graphs).  Entries are never written
    after creation.
    """

    def __init__(self, capacity=64):
        self._entries = OrderedDict()
        self._capacity = capacity

    def __call__(self, batch, length, device):
        key = (str(device), batch, length)
        hit = self._entries.get(key)
        if hit is None:
            hit = torch.arange(batch + 1, dtype=torch.int32, device=device) * length
            self._entries[key] = hit
            if len(self._entries) > self._capacity:
                self._entries.popitem(last=False)
        else:
            self._entries.move_to_end(key)
        return hit


_offsets = _UniformOffsets()


def _check_page_size(k):
    if k.ndim != 4 or k.shape[1] % PAGE_MULTIPLE:
        raise ValueError(f"a paged cache needs [pages, page_size, heads, dim] with page_size a multiple "
                         f"of {PAGE_MULTIPLE}; got shape {tuple(k.shape)}")


def _dense_lse(lse, batch, seqlen):
    """[Hq, B*S] -> [B, Hq, S] (a view)."""
    return lse.reshape(lse.shape[0], batch, seqlen).transpose(0, 1)


def _finish(out, lse, return_lse):
    return (out, lse) if return_lse else out


def flash_attn_varlen_func(
    q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
    dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
    softcap=0.0, alibi_slopes=None, deterministic=False, return_attn_probs=False,
    block_table=None, *, return_softmax_lse=False, out=None,
):
    """Variable-length attention over packed requests.

    q [T, Hq, Dqk]; k/v packed [Tk, Hkv, D] or, with ``block_table`` [B, pages],
    paged [pages, page_size, Hkv, D] (request lengths still come from
    ``cu_seqlens_k``).  Causality is lower-right aligned per request.
    ``deterministic`` fixes the per-row reduction order (one split).
    Returns ``out`` [T, Hq, Dv], plus LSE [Hq, T] with ``return_softmax_lse``.
    """
    reject_training(dropout_p, return_attn_probs, (q, k, v))
    if block_table is not None:
        _check_page_size(k)
    problem = Problem(q, k, v, cu_seqlens_q, max_seqlen_q, max_seqlen_k, cu_k=cu_seqlens_k,
                      table=block_table, scale=softmax_scale, causal=causal, window=tuple(window_size),
                      softcap=softcap, alibi=alibi_slopes, out=out,
                      splits=1 if deterministic else 0, deterministic=deterministic)
    result, lse = solve(problem.validate())
    return _finish(result, lse, return_softmax_lse)


def flash_attn_func(
    q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
    window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
    deterministic=False, return_attn_probs=False, *, return_softmax_lse=False,
):
    """Dense batched attention: q [B, Sq, Hq, Dqk], k/v [B, Sk, Hkv, D].

    Returns ``out`` [B, Sq, Hq, Dv], plus LSE [B, Hq, Sq] with ``return_softmax_lse``.
    """
    if not (q.ndim == k.ndim == v.ndim == 4):
        raise ValueError("dense attention takes 4-D q [B, Sq, Hq, D] and k/v [B, Sk, Hkv, D]")
    if q.shape[0] != k.shape[0] or k.shape[:3] != v.shape[:3]:
        raise ValueError(f"batch/length/head extents disagree: q {tuple(q.shape)}, "
                         f"k {tuple(k.shape)}, v {tuple(v.shape)}")
    batch, sq, sk = q.shape[0], q.shape[1], k.shape[1]
    out, lse = flash_attn_varlen_func(
        q.flatten(0, 1), k.flatten(0, 1), v.flatten(0, 1),
        _offsets(batch, sq, q.device), _offsets(batch, sk, q.device), sq, sk,
        dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
        deterministic, return_attn_probs, return_softmax_lse=True,
    )
    out = out.unflatten(0, (batch, sq))
    return _finish(out, _dense_lse(lse, batch, sq), return_softmax_lse)


def flash_attn_qkvpacked_func(qkv, *args, **kwargs):
    """Dense attention on one packed tensor qkv [B, S, 3, H, D]."""
    if qkv.ndim != 5 or qkv.shape[2] != 3:
        raise ValueError(f"qkv must be [B, S, 3, H, D]; got {tuple(qkv.shape)}")
    q, k, v = qkv.unbind(2)
    return flash_attn_func(q, k, v, *args, **kwargs)


def flash_attn_kvpacked_func(q, kv, *args, **kwargs):
    """Dense attention with q [B, Sq, Hq, D] and kv [B, Sk, 2, Hkv, D]."""
    if kv.ndim != 5 or kv.shape[2] != 2:
        raise ValueError(f"kv must be [B, S, 2, H, D]; got {tuple(kv.shape)}")
    k, v = kv.unbind(2)
    return flash_attn_func(q, k, v, *args, **kwargs)


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, *args, **kwargs):
    """Varlen self-attention on qkv [T, 3, H, D] (queries and keys share offsets)."""
    if qkv.ndim != 4 or qkv.shape[1] != 3:
        raise ValueError(f"qkv must be [T, 3, H, D]; got {tuple(qkv.shape)}")
    q, k, v = qkv.unbind(1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen, *args, **kwargs)


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                    *args, **kwargs):
    """Varlen attention with q [T, Hq, D] and kv [Tk, 2, Hkv, D]."""
    if kv.ndim != 4 or kv.shape[1] != 2:
        raise ValueError(f"kv must be [T, 2, H, D]; got {tuple(kv.shape)}")
    k, v = kv.unbind(1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                  *args, **kwargs)


def _cache_lengths(cache_seqlens, batch, k_new, table, capacity, device):
    """cache_seqlens as an int32 [B] device tensor (the caller's, never modified)."""
    if cache_seqlens is None:
        if k_new is not None or table is not None:
            raise ValueError("cache_seqlens is required to append to a cache or to read a paged one")
        cache_seqlens = capacity
    if isinstance(cache_seqlens, int):
        return torch.full((batch,), cache_seqlens, dtype=torch.int32, device=device)
    if (not torch.is_tensor(cache_seqlens) or tuple(cache_seqlens.shape) != (batch,)
            or cache_seqlens.dtype != torch.int32 or cache_seqlens.device != device):
        raise ValueError(f"cache_seqlens must be an int or an int32 [{batch}] tensor on {device}")
    return cache_seqlens


def flash_attn_with_kvcache(
    q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
    cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None, block_table=None,
    softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
    rotary_interleaved=True, alibi_slopes=None, num_splits=0,
    return_softmax_lse=False,
):
    """Attention of q [B, Sq, Hq, D] over a KV cache, optionally appending first.

    The cache is dense [rows, capacity, Hkv, D] (request b reads row
    ``cache_batch_idx[b]``, default b) or paged [pages, page_size, Hkv, D]
    through ``block_table``.  ``cache_seqlens`` are the lengths before the
    append and are never modified; new k/v [B, Snew, Hkv, D] land at
    ``cache_seqlens[b] + j`` (after an optional rotary embedding of q and k).
    ``cache_leftpad`` hides the first positions of a dense cache row from
    attention without moving where appends go.
    Returns ``out`` [B, Sq, Hq, Dv], plus LSE [B, Hq, Sq] with ``return_softmax_lse``.
    """
    reject_training(0.0, False, (q, k, v, k_cache, v_cache))
    if not (q.ndim == k_cache.ndim == v_cache.ndim == 4):
        raise ValueError("q and both caches must be 4-D")
    if (k is None) != (v is None):
        raise ValueError("new k and v come together")
    if block_table is not None:
        if cache_leftpad is not None:
            raise ValueError("cache_leftpad applies to dense caches only, not to a block_table")
        _check_page_size(k_cache)
    batch, sq = q.shape[0], q.shape[1]
    lengths = _cache_lengths(cache_seqlens, batch, k, block_table, k_cache.shape[1], q.device)
    if (rotary_cos is None) != (rotary_sin is None):
        raise ValueError("rotary_cos and rotary_sin come together")
    if rotary_cos is not None:
        if k is None:
            raise ValueError("a rotary embedding is applied to new k/v only; none were given")
        from ._cache import rotary
        q, k = rotary(q, k, rotary_cos, rotary_sin, lengths, rotary_interleaved=rotary_interleaved,
                      causal=causal, window_size=window_size)
    if k is not None:
        if k.ndim != 4 or v.ndim != 4 or k.shape[0] != batch or v.shape[:3] != k.shape[:3]:
            raise ValueError(f"new k {tuple(k.shape)} / v {tuple(v.shape)} must be [{batch}, Snew, Hkv, D]")
        from ._cache import append_kvcache
        append_kvcache(k, v, k_cache, v_cache, lengths, cache_batch_idx=cache_batch_idx,
                       cache_leftpad=cache_leftpad, block_table=block_table)
        lengths = lengths + k.shape[1]
    if block_table is not None:
        # Table rows follow the query batch; cache_batch_idx only remaps dense rows.
        table, max_k = block_table, block_table.shape[1] * k_cache.shape[1]
    else:
        rows = cache_batch_idx if cache_batch_idx is not None else torch.arange(batch, device=q.device)
        table, max_k = rows.to(torch.int32).reshape(batch, 1), k_cache.shape[1]
    if cache_leftpad is not None:
        lengths = lengths - cache_leftpad
    problem = Problem(q.flatten(0, 1), k_cache, v_cache, _offsets(batch, sq, q.device), sq, max_k,
                      used_k=lengths, table=table, leftpad=cache_leftpad, scale=softmax_scale,
                      causal=causal, window=tuple(window_size), softcap=softcap, alibi=alibi_slopes,
                      splits=num_splits)
    out, lse = solve(problem.validate())
    out = out.unflatten(0, (batch, sq))
    return _finish(out, _dense_lse(lse, batch, sq), return_softmax_lse)
