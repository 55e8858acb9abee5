"""Split-KV decode on gfx950 (counterpart of flash_attn_mps/_decode.py:40-99): one
query row per request, and 2..16 rows per request (speculative decode) on the
matrix-core kernel.

The split plan uses only host-known sizes: the most keys a query can see
(max_seqlen_k clipped by a left window, _decode.py:63; with R rows the first
row's window, R - 1 keys wider) and the number of (request, query-head group)
work units.  A split covers `span` keys; the span
starts at 4096 and halves (down to 128) until the grid holds at least 1024
workgroups (two rounds of the 512 that the decode kernels keep resident),
so small batches still fill the 256 compute units.  (With the kernels'
longest-first work order, 4096-key spans beat 2048: config 3 0.749-0.765
-> 0.730 ms, its 4-row step 0.79-0.80 -> 0.755, config 5 -1%; and 1024
workgroups beat 2048: config 4's single split 0.324-0.328 -> 0.318 ms.)  An explicit
num_splits is honoured.  fa_decode_fwd_noalloc plans the same way in C.
"""
import torch

from . import _lib
from ._attention import _partials, build_args

_MIN_WORKGROUPS = 1024
_START_SPAN = 4096
_MIN_SPAN = 128
_SPAN_ALIGN = 32


def split_plan(batch, head_groups, visible, num_splits):
    """(splits, span) covering `visible` keys per request: splits * span >= visible."""
    if visible <= 0:
        return 1, _SPAN_ALIGN
    if num_splits:
        span = -(-visible // num_splits)
        span = max(_SPAN_ALIGN, -(-span // _SPAN_ALIGN) * _SPAN_ALIGN)
        return max(1, min(num_splits, -(-visible // span))), span
    span = _START_SPAN
    while span > _MIN_SPAN and batch * head_groups * -(-visible // span) < _MIN_WORKGROUPS:
        span //= 2
    return -(-visible // span), span


# Head dims that run zero-padded inside a larger decode tile.
_TILE_DIM = {32: 64, 72: 128, 80: 128, 96: 128}


def group_tile(heads, kv_heads, dim_qk, dim_v):
    """Query heads per decode workgroup; mirrors decode_group_tile() in decode_kernel.hip."""
    group = heads // kv_heads
    chunks = (_TILE_DIM.get(dim_qk, dim_qk) + _TILE_DIM.get(dim_v, dim_v)) // 16
    most = 8 if chunks == 16 else 1
    while most < 4 and 2 * most * chunks <= 64:
        most *= 2
    tiles = -(-group // most)
    tile = 1
    while -(-group // tile) > tiles:
        tile *= 2
    return tile


# The matrix-core decode (decode_gqa.h): one query row per request from
# DECODE_GQA_MIN_GROUP query heads per KV head (any group when 64-dim KV heads
# run in pairs, gqa_pack), or 2..DECODE_GQA_MAX_ROWS rows per request with any
# group (decode_kernel.h); its workgroups take 32 columns, i.e. 32 // rows
# query heads.
_GQA_MIN_GROUP = 3
_GQA_MAX_ROWS = 16


def uses_gqa_kernel(p, rows=None):
    """Whether fa_decode_fwd runs Problem `p` with `rows` query rows per
    request (default p.max_q) on the matrix-core GQA kernel (mirrors
    pick_decode_gqa in decode_gqa.hip, stride alignment aside, which only
    changes the split plan's workgroup estimate)."""
    page = p.k.shape[1] if p.paged else 0
    rows = p.max_q if rows is None else rows
    small = p.dim_qk == 64 and gqa_pack(p, 1) == 2   # paired 64-dim heads take groups of 1-2 too
    rows_ok = (p.heads // p.kv_heads >= _GQA_MIN_GROUP or small) if rows <= 1 else rows <= _GQA_MAX_ROWS
    out_dtype = p.out.dtype if p.out is not None else p.output_dtype
    return (rows_ok and p.q.dtype in (torch.float16, torch.bfloat16) and out_dtype == p.q.dtype
            and p.k.dtype == p.v.dtype and p.k.dtype in (p.q.dtype, torch.float8_e4m3fn)
            and p.dim_qk == p.dim_v and p.dim_qk in (64, 128) and p.alibi is None and p.mask is None
            and page % 16 == 0)


def gqa_pack(p, rows=1):
    """KV heads per matrix-core decode workgroup at `rows` query rows per
    request (mirrors packable() in decode_gqa.hip): 2 when 64-dim heads (or
    128-dim E4M3 heads) sit next to each other in every key row (head stride
    = the head dim, rows of two heads or more), the KV heads pair up, both
    heads' query columns fit one 32-column tile, and the cache is E4M3 or has
    8 or more KV heads; else 1."""
    k, v, d = p.k, p.v, p.dim_qk
    fp8 = k.dtype == torch.float8_e4m3fn
    fits = 2 * (p.heads // p.kv_heads) * max(rows, 1) <= 32
    return 2 if ((d == 64 or (d == 128 and fp8)) and p.dim_v == d and p.kv_heads % 2 == 0 and k.stride(-2) == d
                 and v.stride(-2) == d and k.stride(-3) >= 2 * d and v.stride(-3) >= 2 * d and fits
                 and (fp8 or p.kv_heads >= 8)) else 1


def valu_pair(p):
    """KV heads per VALU-decode workgroup (mirrors valu_pair() in
    decode_kernel.hip): 2 when neighbouring heads' rows sit next to each other
    in every key row, there are 8 or more KV heads and no ALiBi, for E4M3
    d128 caches (groups of 1-2) and 16-bit 192/128 (groups of 1), unless the
    call runs one split per request; else 1."""
    k, v, dq, dv = p.k, p.v, p.dim_qk, p.dim_v
    if p.splits == 1:
        return 1
    fp8 = k.dtype == torch.float8_e4m3fn
    e4m3_128 = fp8 and dq == 128 and dv == 128
    diffkv = not fp8 and (dq, dv) == (192, 128)
    if p.alibi is not None or not (e4m3_128 or diffkv):
        return 1
    if (p.kv_heads % 2 or k.stride(-2) != dq or v.stride(-2) != dv or k.stride(-3) < 2 * dq
            or v.stride(-3) < 2 * dv or p.kv_heads < 8):
        return 1
    return 2 if p.heads // p.kv_heads <= (1 if diffkv else 2) else 1


def workgroups_per_token(heads, kv_heads, dim_qk, dim_v, gqa=False, rows=1, pack=1):
    """Decode workgroups per (request, split): KV heads x ceil(group / tile);
    either kernel takes `pack` KV heads (and their query heads) per
    workgroup (the VALU kernel then holds the pair's heads in one tile)."""
    group = heads // kv_heads
    if gqa:
        return kv_heads // pack * -(-(pack * group) // (32 // max(rows, 1)))
    if pack == 2:
        return kv_heads // 2
    return kv_heads * -(-group // group_tile(heads, kv_heads, dim_qk, dim_v))


def decode_workgroups(p, rows=1):
    """Decode workgroups per (request, split) of Problem `p` at `rows` query
    rows per request (mirrors decode_head_groups in decode_kernel.hip)."""
    gqa = uses_gqa_kernel(p, rows)
    pack = gqa_pack(p, rows) if gqa else valu_pair(p)
    return workgroups_per_token(p.heads, p.kv_heads, p.dim_qk, p.dim_v, gqa, rows, pack)


def decode(p, out, splits=None):
    """One query per request of Problem `p` (cu_seqlens_q steps of 0 or 1);
    `splits` overrides the split count (1: the fixed-order route).

    Returns (out, lse).  The split-KV kernels handle 16-bit queries over
    16-bit or FP8 caches at their compiled head dims; other dtype/dim/stride
    combinations run the generic kernel with the reference's split rule
    (_decode.py:63-64).
    """
    lse = torch.empty((p.heads, p.tokens), dtype=torch.float32, device=p.device)
    a = build_args(p, out, lse, max_q=1)
    a.causal, a.causal_by_batch = 0, None   # a right-aligned single query has no future keys
    if _run_split_kv(p, a, 1, splits):
        return out, lse
    splits = splits or p.splits or max(1, min(32, -(-p.visible_max // 256)))
    if splits > 1:
        _partials(p, a, (splits, p.tokens, p.heads, p.dim_v), (splits, p.heads, p.tokens))
    a.num_splits = splits
    _lib.call("fa_attn_fwd", a, p.device)
    return out, lse


def decode_rows(p, out):
    """2..16 query rows per request (speculative / multi-token decode): the
    matrix-core decode with (head, row) columns, split over the keys like the
    one-row decode.  Each request's rows are its last key positions.  Returns
    (out, lse), or None (nothing launched) when the kernel does not take the
    arguments."""
    if not uses_gqa_kernel(p):
        return None
    lse = torch.empty((p.heads, p.tokens), dtype=torch.float32, device=p.device)
    a = build_args(p, out, lse)
    return (out, lse) if _run_split_kv(p, a, p.max_q) else None


def _run_split_kv(p, a, rows, splits=None):
    """fa_decode_fwd with the split plan (or `splits` splits) and partials
    (outputs [batch][S][rows][Hq][Dv], LSEs [batch][rows][Hq][S]); False when
    the decode kernels do not take the arguments."""
    if not _lib.supported("fa_decode_supported", a):
        return False
    groups = decode_workgroups(p, rows)
    left = p.window[0]
    visible = min(p.max_k, left + rows) if left >= 0 else p.max_k   # the first row's window
    splits, span = split_plan(p.batch, groups, visible, splits or p.splits)
    a.num_splits, a.split_span = splits, span
    if splits > 1:
        _partials(p, a, (p.batch, splits, rows, p.heads, p.dim_v), (p.batch, rows, p.heads, splits))
    _lib.call("fa_decode_fwd", a, p.device)
    return True
