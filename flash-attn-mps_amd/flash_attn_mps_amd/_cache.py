"""Cache scatter, FA2 append and rotary embedding on gfx950.

Host side of fa_store_kvcache / fa_append_kvcache / fa_rotary; mirrors
flash_attn_mps/_cache.py:67-155 (argument checks, scalar-or-per-head FP8
scales, lengths broadcast, RoPE position rules) with the kernels of
csrc/cache_kernels.hip.
"""
from functools import lru_cache

import torch

from . import _lib


def _gpu(*tensors):
    if any(t.device.type != "cuda" for t in tensors if t is not None):
        raise ValueError("operations require GPU (HIP) tensors")


@lru_cache(maxsize=None)
def _unit_scale(device):
    return torch.ones(1, device=device, dtype=torch.float32)


def _scale(scale, heads, device):
    """flash_attn_mps/_cache.py:55-59: scalar or one value per KV head, fp32."""
    if scale is None:
        scale = _unit_scale(device)
    else:
        scale = torch.as_tensor(scale, device=device, dtype=torch.float32)
    if scale.numel() not in (1, heads):
        raise ValueError("scale must be scalar or have one value per KV head")
    return scale.reshape(-1).contiguous(), 0 if scale.numel() == 1 else 1


def _store_code(x, cache):
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("input dtype must be float16, bfloat16 or float32")
    if cache.dtype != torch.float8_e4m3fn and cache.dtype != x.dtype:
        raise TypeError("cache dtype must match input or be float8_e4m3fn")
    return _lib.DTYPE_CODE[x.dtype], _lib.DTYPE_CODE[cache.dtype]


def _desc(x, cache, scale, tensor_strides, keep):
    d = _lib.StoreDesc()
    xc, cc = _store_code(x, cache)
    d.x, d.cache = x.data_ptr(), cache.data_ptr()
    d.x_dtype, d.cache_dtype = xc, cc
    d.heads, d.dim = x.shape[-2], x.shape[-1]
    d.x_stride[:] = tensor_strides
    d.cache_stride[:] = list(cache.stride())
    if cache.dtype == torch.float8_e4m3fn:
        s, stride = _scale(scale, x.shape[-2], x.device)
        keep.append(s)
        d.scale, d.scale_stride = s.data_ptr(), stride
    return d


def store_kvcache(k, v, k_cache, v_cache, slot_mapping, *, k_scale=None, v_scale=None):
    """Scatter [tokens, heads, dim] K/V into physical cache slots; -1 skips."""
    _gpu(k, v, k_cache, v_cache, slot_mapping)
    if k.ndim != 3 or v.ndim != 3 or k.shape[:2] != v.shape[:2]:
        raise ValueError("K/V must have matching [tokens, heads, dim] shapes")
    if (slot_mapping.ndim != 1 or slot_mapping.numel() != k.shape[0]
            or slot_mapping.dtype not in (torch.int32, torch.int64)):
        raise ValueError("slot_mapping must be int32/int64 with one slot per token")
    for x, cache in ((k, k_cache), (v, v_cache)):
        if cache.ndim != 4 or cache.shape[2:] != x.shape[1:]:
            raise ValueError("cache must have shape [blocks, block_size, heads, dim]")
    if k_cache.shape[:2] != v_cache.shape[:2]:
        raise ValueError("K and V caches must have the same pages and page size")
    keep = []
    args = _lib.StoreArgs()
    pairs = [(x, c, s) for x, c, s in ((k, k_cache, k_scale), (v, v_cache, v_scale)) if x.numel()]
    if not pairs or k.shape[0] == 0:
        return
    for i, (x, c, s) in enumerate(pairs):
        args.kv[i] = _desc(x, c, s, list(x.stride()), keep)
    args.slots = slot_mapping.data_ptr()
    args.slot_dtype = _lib.I64 if slot_mapping.dtype == torch.int64 else _lib.I32
    args.slot_stride = slot_mapping.stride(0)
    args.tokens = k.shape[0]
    args.page_size = k_cache.shape[1]
    args.num_pages = k_cache.shape[0]
    _lib.call("fa_store_kvcache", args, k.device)


def _integers(value, count, device):
    if value is None:
        value = 0
    value = torch.as_tensor(value, dtype=torch.int32, device=device)
    if value.numel() == 1:
        value = value.reshape(1).expand(count)
    if value.numel() != count:
        raise ValueError(f"expected {count} integer values")
    return value.contiguous()


def append_kvcache(k, v, k_cache, v_cache, cache_seqlens, *, cache_batch_idx=None,
                   cache_leftpad=None, block_table=None, k_scale=None, v_scale=None):
    """Append [batch, new_tokens, heads, dim] K/V at cache_seqlens[b] + j without
    changing the lengths (flash_attn_mps/_cache.py:99-127)."""
    _gpu(k, v, k_cache, v_cache, block_table)
    if k.ndim != 4 or v.ndim != 4 or k.shape[:3] != v.shape[:3]:
        raise ValueError("K/V must have matching [batch, new_tokens, heads, dim] shapes")
    batch = k.shape[0]
    lengths = _integers(cache_seqlens, batch, k.device)
    remap = block_table is None and cache_batch_idx is not None
    indices = _integers(cache_batch_idx, batch, k.device) if remap else None
    # FA2 lengths are physical exclusive ends that already include left padding,
    # so new tokens go to length + j, never length + leftpad + j.
    if cache_leftpad is not None:
        _integers(cache_leftpad, batch, k.device)
    if block_table is not None and block_table.ndim != 2:
        raise ValueError("block_table must have shape [cache_batch, blocks_per_sequence]")
    table = None if block_table is None else block_table.to(torch.int32).contiguous()
    for x, cache in ((k, k_cache), (v, v_cache)):
        if cache.ndim != 4 or cache.shape[2:] != x.shape[2:]:
            raise ValueError("cache must have shape [rows, capacity, heads, dim]")
    keep = [lengths, indices, table]
    pairs = [(x, c, s) for x, c, s in ((k, k_cache, k_scale), (v, v_cache, v_scale)) if x.numel()]
    if not pairs:
        return
    args = _lib.AppendArgs()
    for i, (x, c, s) in enumerate(pairs):
        args.kv[i] = _desc(x, c, s, list(x.stride())[1:], keep)
        args.x_batch_stride[i] = x.stride(0)
    args.lengths = lengths.data_ptr()
    args.batch_index = _lib.ptr(indices)
    args.block_table = _lib.ptr(table)
    args.batch, args.new_tokens = batch, k.shape[1]
    args.page_size, args.num_blocks = k_cache.shape[1], k_cache.shape[0]
    args.table_rows = 0 if table is None else table.shape[0]
    args.table_cols = 0 if table is None else table.shape[1]
    _lib.call("fa_append_kvcache", args, k.device)


def rotary(q, k, cos, sin, cache_seqlens, *, rotary_interleaved=True, causal=False,
           window_size=(-1, -1)):
    """Rotate new K at old_length + j and Q at its causal/local absolute position
    (flash_attn_mps/_cache.py:130-155); returns new contiguous tensors."""
    _gpu(q, k, cos, sin)
    if q.ndim != 4 or (k is not None and (k.ndim != 4 or q.shape[0] != k.shape[0])):
        raise ValueError("Q/K must have shape [batch, tokens, heads, dim]")
    if cos.ndim != 2 or sin.shape != cos.shape or cos.shape[1] * 2 > q.shape[-1]:
        raise ValueError("rotary cosine/sine must have shape [positions, rotary_dim/2]")
    cosine, sine = cos.float().contiguous(), sin.float().contiguous()
    lengths = _integers(cache_seqlens, q.shape[0], q.device)
    outputs = []
    for x, advance in ((q, causal or tuple(window_size) != (-1, -1)), (k, True)):
        if x is None:
            outputs.append(None)
            continue
        if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise TypeError("rotary supports float16, bfloat16 and float32")
        if cos.shape[1] * 2 > x.shape[-1]:
            raise ValueError("rotary dimension exceeds head dimension")
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        if x.numel():
            args = _lib.RotaryArgs()
            args.x, args.out = x.data_ptr(), output.data_ptr()
            args.cos_table, args.sin_table = cosine.data_ptr(), sine.data_ptr()
            args.lengths = lengths.data_ptr()
            args.dtype = _lib.DTYPE_CODE[x.dtype]
            args.interleaved, args.advance = int(rotary_interleaved), int(bool(advance))
            args.batch, args.seq, args.heads, args.dim = x.shape
            args.half_rot, args.table_rows = cos.shape[1], cos.shape[0]
            args.x_stride[:] = list(x.stride())
            _lib.call("fa_rotary", args, x.device)
        outputs.append(output)
    return tuple(outputs)
