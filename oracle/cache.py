"""TEST INFRASTRUCTURE ONLY: CPU restatement of the cache kernels.

store_kvcache restates flash_attn_mps/kernels/cache.metal:20-39 with the host
rules of flash_attn_mps/_cache.py:55-85: cache[slot // P, slot % P, h, :] =
x[t, h, :] for 0 <= slot < pages * P, raw bits for an equal dtype and
E4M3FN(x / scale[h]) for an FP8 cache.  append_kvcache restates
cache.metal:41-56 (position lengths[b] + j, batch remap or page table,
out-of-range skipped) and rotary cache.metal:58-76 (interleaved or split
halves, position lengths[b] + (j if advance else 0)).
"""
import numpy as np
import torch

from . import fp8


def _fp8_codes(x, scale, heads):
    """x [..., H, D] -> uint8 codes of float32(x) / scale[h] (IEEE fp32 division)."""
    xs = x.detach().cpu().float().contiguous()
    shape = xs.shape
    s = torch.ones(1) if scale is None else torch.as_tensor(scale, dtype=torch.float32).reshape(-1).cpu()
    codes = fp8.encode_scaled(xs.reshape(-1, heads, shape[-1]).numpy(), s.numpy())
    return torch.from_numpy(codes).reshape(shape)


def store_kvcache(x, cache, slots, scale=None):
    """Return a CPU copy of `cache` after storing x [T, H, D] at `slots`."""
    cache = cache.detach().cpu().clone()
    slots = [int(s) for s in slots.detach().cpu().tolist()]
    pages, page = cache.shape[0], cache.shape[1]
    fp8_cache = cache.dtype == torch.float8_e4m3fn
    values = _fp8_codes(x, scale, x.shape[1]) if fp8_cache else x.detach().cpu()
    raw = cache.view(torch.uint8) if fp8_cache else cache
    for t, slot in enumerate(slots):
        if slot < 0 or slot >= pages * page:
            continue
        raw[slot // page, slot % page] = values[t]
    return cache


def append_kvcache(x, cache, lengths, batch_index=None, block_table=None, scale=None):
    """Return a CPU copy of `cache` after appending x [B, S, H, D] at lengths[b] + j."""
    cache = cache.detach().cpu().clone()
    batch, new = x.shape[:2]
    lengths = [int(v) for v in torch.as_tensor(lengths).reshape(-1).expand(batch).tolist()]
    fp8_cache = cache.dtype == torch.float8_e4m3fn
    values = _fp8_codes(x, scale, x.shape[2]) if fp8_cache else x.detach().cpu()
    raw = cache.view(torch.uint8) if fp8_cache else cache
    table = None if block_table is None else block_table.detach().cpu().long()
    rows = cache.shape[0] if table is None else table.shape[0]
    capacity = cache.shape[1]
    for b in range(batch):
        row = b if (table is not None or batch_index is None) else int(batch_index.reshape(-1)[b])
        for j in range(new):
            pos = lengths[b] + j
            limit = table.shape[1] * capacity if table is not None else capacity
            if row < 0 or row >= rows or pos < 0 or pos >= limit:
                continue
            block = int(table[row, pos // capacity]) if table is not None else row
            offset = pos % capacity if table is not None else pos
            if block < 0 or block >= cache.shape[0]:
                continue
            raw[block, offset] = values[b, j]
    return cache


def rotary(x, cos, sin, lengths, interleaved, advance):
    """Rotate x [B, S, H, D] (float64 result); cos/sin [positions, rot/2]."""
    x = x.detach().cpu().double()
    cos = cos.detach().cpu().double()
    sin = sin.detach().cpu().double()
    half = cos.shape[1]
    out = x.clone()
    lengths = [int(v) for v in torch.as_tensor(lengths).reshape(-1).tolist()]
    for b in range(x.shape[0]):
        for j in range(x.shape[1]):
            p = lengths[b] + (j if advance else 0)
            c, s = cos[p], sin[p]
            if interleaved:
                a, z = x[b, j, :, 0:2 * half:2], x[b, j, :, 1:2 * half:2]
            else:
                a, z = x[b, j, :, :half], x[b, j, :, half:2 * half]
            first, second = a * c - z * s, z * c + a * s
            if interleaved:
                out[b, j, :, 0:2 * half:2], out[b, j, :, 1:2 * half:2] = first, second
            else:
                out[b, j, :, :half], out[b, j, :, half:2 * half] = first, second
    return out
