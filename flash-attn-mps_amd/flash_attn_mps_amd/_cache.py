"""KV-cache writes and rotary embedding on gfx950: host side of
fa_store_kvcache / fa_append_kvcache / fa_rotary (counterpart of
flash_attn_mps/_cache.py:55-155).

* store_kvcache scatters token rows to physical slots (page = slot // P,
  row = slot % P); negative or out-of-range slots are skipped by the kernel.
* append_kvcache writes new rows at ``lengths[b] + j`` of a dense cache row
  or through a page table; the lengths themselves are not touched.
* An FP8 (E4M3FN) cache stores E4M3(x / scale) with scale a scalar or one
  value per KV head; 16-bit and fp32 caches of the input's dtype get the
  input's bits.
"""
from functools import lru_cache

import torch

from . import _lib
from ._problem import on_gpu

_INPUT_TYPES = (torch.float16, torch.bfloat16, torch.float32)


def _require_gpu(**tensors):
    for name, t in tensors.items():
        if t is not None and not on_gpu(t):
            raise ValueError(f"{name} is on {t.device}; cache operations run on a ROCm GPU")


@lru_cache(maxsize=None)
def _one(device):
    """A resident fp32 1.0 per device: the FP8 scale when the caller gives none."""
    return torch.ones(1, dtype=torch.float32, device=device)


def _per_head_scale(scale, heads, device):
    """(fp32 tensor, stride): stride 0 shares one scale, 1 reads one per head."""
    t = _one(device) if scale is None else torch.as_tensor(scale, dtype=torch.float32, device=device)
    if t.numel() == 1:
        return t.reshape(1), 0
    if t.numel() == heads:
        return t.reshape(heads).contiguous(), 1
    raise ValueError(f"an FP8 scale is one value or one per KV head ({heads}); got {t.numel()} values")


def _per_request(value, count, device, name):
    """An int32 [count] device tensor from an int, a 1-element or a [count] tensor."""
    t = torch.as_tensor(0 if value is None else value, dtype=torch.int32, device=device)
    if t.numel() == 1:
        t = t.reshape(1).expand(count)
    if t.numel() != count:
        raise ValueError(f"{name}: expected 1 or {count} values, got {t.numel()}")
    return t.contiguous()


def _write_desc(x, cache, scale, x_strides, keep):
    """fa_store_desc for writing `x` rows into `cache` (checks the dtype pair)."""
    if x.dtype not in _INPUT_TYPES:
        raise TypeError(f"cache inputs are float16, bfloat16 or float32; got {x.dtype}")
    fp8 = cache.dtype == torch.float8_e4m3fn
    if not fp8 and cache.dtype != x.dtype:
        raise TypeError(f"a {cache.dtype} cache cannot take {x.dtype} rows (use the same dtype or float8_e4m3fn)")
    d = _lib.StoreDesc()
    d.x, d.cache = x.data_ptr(), cache.data_ptr()
    d.x_dtype, d.cache_dtype = _lib.DTYPE_CODE[x.dtype], _lib.DTYPE_CODE[cache.dtype]
    d.heads, d.dim = x.shape[-2], x.shape[-1]
    d.x_stride[:] = x_strides
    d.cache_stride[:] = cache.stride()
    if fp8:
        s, stride = _per_head_scale(scale, x.shape[-2], x.device)
        keep.append(s)
        d.scale, d.scale_stride = s.data_ptr(), stride
    return d


def _check_cache_shape(x, cache, row_dims):
    """cache [pages, page_size, heads, dim] matching the (heads, dim) of x."""
    if cache.ndim != 4 or tuple(cache.shape[2:]) != tuple(x.shape[row_dims:]):
        raise ValueError(f"cache {tuple(cache.shape)} must be [pages, page_size, {x.shape[-2]}, {x.shape[-1]}]")


def store_kvcache(k, v, k_cache, v_cache, slot_mapping, *, k_scale=None, v_scale=None):
    """Write k/v [T, Hkv, D] to the cache slots slot_mapping [T] (int32/int64)."""
    _require_gpu(k=k, v=v, k_cache=k_cache, v_cache=v_cache, slot_mapping=slot_mapping)
    if k.ndim != 3 or v.ndim != 3 or k.shape[:2] != v.shape[:2]:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must be [tokens, heads, dim] "
                         "with the same tokens and heads")
    if (slot_mapping.ndim != 1 or slot_mapping.numel() != k.shape[0]
            or slot_mapping.dtype not in (torch.int32, torch.int64)):
        raise ValueError(f"slot_mapping must be int32/int64 with one entry per token ({k.shape[0]})")
    _check_cache_shape(k, k_cache, 1)
    _check_cache_shape(v, v_cache, 1)
    if k_cache.shape[:2] != v_cache.shape[:2]:
        raise ValueError("the K and V caches must have the same pages and page size")
    writes = [(x, c, s) for x, c, s in ((k, k_cache, k_scale), (v, v_cache, v_scale)) if x.numel()]
    if not writes:
        return
    keep = []
    args = _lib.StoreArgs()
    for i, (x, c, s) in enumerate(writes):
        args.kv[i] = _write_desc(x, c, s, x.stride(), keep)
    args.slots = slot_mapping.data_ptr()
    args.slot_dtype = _lib.I64 if slot_mapping.dtype == torch.int64 else _lib.I32
    args.slot_stride = slot_mapping.stride(0)
    args.tokens, args.page_size, args.num_pages = k.shape[0], k_cache.shape[1], k_cache.shape[0]
    _lib.call("fa_store_kvcache", args, k.device)


def append_kvcache(k, v, k_cache, v_cache, cache_seqlens, *, cache_batch_idx=None,
                   cache_leftpad=None, block_table=None, k_scale=None, v_scale=None):
    """Write k/v [B, Snew, Hkv, D] at position cache_seqlens[b] + j of request b.

    Dense caches [rows, capacity, Hkv, D] take row ``cache_batch_idx[b]``
    (default b); with ``block_table`` [rows, pages] the position goes through
    the table.  cache_leftpad does not move the write: FA2 lengths already
    count the padding (flash_attn_mps/_cache.py:99-127).
    """
    _require_gpu(k=k, v=v, k_cache=k_cache, v_cache=v_cache, block_table=block_table)
    if k.ndim != 4 or v.ndim != 4 or k.shape[:3] != v.shape[:3]:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must be [batch, new_tokens, heads, dim] "
                         "with the same batch, tokens and heads")
    batch = k.shape[0]
    lengths = _per_request(cache_seqlens, batch, k.device, "cache_seqlens")
    rows = None
    if block_table is None and cache_batch_idx is not None:
        rows = _per_request(cache_batch_idx, batch, k.device, "cache_batch_idx")
    if cache_leftpad is not None:
        _per_request(cache_leftpad, batch, k.device, "cache_leftpad")
    if block_table is not None and block_table.ndim != 2:
        raise ValueError(f"block_table must be [rows, pages]; got {tuple(block_table.shape)}")
    table = None if block_table is None else block_table.to(torch.int32).contiguous()
    _check_cache_shape(k, k_cache, 2)
    _check_cache_shape(v, v_cache, 2)
    writes = [(x, c, s) for x, c, s in ((k, k_cache, k_scale), (v, v_cache, v_scale)) if x.numel()]
    if not writes:
        return
    keep = [lengths, rows, table]
    args = _lib.AppendArgs()
    for i, (x, c, s) in enumerate(writes):
        args.kv[i] = _write_desc(x, c, s, x.stride()[1:], keep)
        args.x_batch_stride[i] = x.stride(0)
    args.lengths = lengths.data_ptr()
    args.batch_index = _lib.ptr(rows)
    args.block_table = _lib.ptr(table)
    args.batch, args.new_tokens = batch, k.shape[1]
    args.page_size, args.num_blocks = k_cache.shape[1], k_cache.shape[0]
    args.table_rows, args.table_cols = (0, 0) if table is None else tuple(table.shape)
    _lib.call("fa_append_kvcache", args, k.device)


def rotary(q, k, cos, sin, cache_seqlens, *, rotary_interleaved=True, causal=False, window_size=(-1, -1)):
    """Rotary embedding of q [B, Sq, Hq, D] and new k [B, Snew, Hkv, D] (fresh tensors).

    cos/sin are [positions, rotary_dim / 2]; the first rotary_dim dims rotate
    as interleaved pairs (2i, 2i+1) or as halves (i, i + rotary_dim / 2).  New
    key j sits at cache_seqlens[b] + j; queries advance with j only for causal
    or local attention, else all sit at cache_seqlens[b]
    (flash_attn_mps/_cache.py:130-155).  A position past the table rotates to NaN.
    """
    _require_gpu(q=q, k=k, cos=cos, sin=sin)
    if q.ndim != 4 or (k is not None and (k.ndim != 4 or k.shape[0] != q.shape[0])):
        raise ValueError("q and k must be [batch, tokens, heads, dim] with one batch")
    if cos.ndim != 2 or sin.shape != cos.shape or 2 * cos.shape[1] > q.shape[-1]:
        raise ValueError(f"cos/sin must be [positions, rotary_dim / 2] with rotary_dim <= {q.shape[-1]}; "
                         f"got {tuple(cos.shape)} / {tuple(sin.shape)}")
    cos32, sin32 = cos.float().contiguous(), sin.float().contiguous()
    lengths = _per_request(cache_seqlens, q.shape[0], q.device, "cache_seqlens")
    query_moves = bool(causal) or tuple(window_size) != (-1, -1)
    rotated = []
    for x, advance in ((q, query_moves), (k, True)):
        if x is None:
            rotated.append(None)
            continue
        if x.dtype not in _INPUT_TYPES:
            raise TypeError(f"rotary embedding takes float16, bfloat16 or float32; got {x.dtype}")
        if 2 * cos.shape[1] > x.shape[-1]:
            raise ValueError(f"rotary_dim {2 * cos.shape[1]} exceeds the head dim {x.shape[-1]}")
        y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        if x.numel():
            a = _lib.RotaryArgs()
            a.x, a.out = x.data_ptr(), y.data_ptr()
            a.cos_table, a.sin_table, a.lengths = cos32.data_ptr(), sin32.data_ptr(), lengths.data_ptr()
            a.dtype = _lib.DTYPE_CODE[x.dtype]
            a.interleaved, a.advance = int(bool(rotary_interleaved)), int(advance)
            a.batch, a.seq, a.heads, a.dim = x.shape
            a.half_rot, a.table_rows = cos.shape[1], cos.shape[0]
            a.x_stride[:] = x.stride()
            _lib.call("fa_rotary", a, x.device)
        rotated.append(y)
    return tuple(rotated)
