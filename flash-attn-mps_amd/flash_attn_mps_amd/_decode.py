"""Single-token attention with grouped KV reads and split-KV reduction on gfx950.

Counterpart of flash_attn_mps/_decode.py:40-99.  The split plan uses only
host-known sizes: the effective maximum key count (clipped by a left window,
_decode.py:63) and the number of (request, head-group) work units.  A split
covers `span` keys; the default span starts at 2048 keys and halves (down to
128) until the grid holds at least 2048 workgroups, so small batches still
fill the 256 compute units.  An explicit num_splits is honoured.
"""
import torch

from . import _lib
from ._attention import build_args

_MIN_WORKGROUPS = 2048
_START_SPAN = 2048
_MIN_SPAN = 128


def _round_up(x, m):
    return (x + m - 1) // m * m


def split_plan(batch, head_groups, effective_max, num_splits):
    """Return (splits, span) for `effective_max` keys per request."""
    if effective_max <= 0:
        return 1, 32
    if num_splits:
        span = max(32, _round_up(-(-effective_max // num_splits), 32))
        return max(1, min(num_splits, -(-effective_max // span))), span
    span = _START_SPAN
    while span > _MIN_SPAN and batch * head_groups * -(-effective_max // span) < _MIN_WORKGROUPS:
        span //= 2
    return -(-effective_max // span), span


def _tile_dim(d):
    """Head dim of the decode tile a tensor head dim runs in (decode_tile_dim)."""
    return {32: 64, 72: 128, 80: 128, 96: 128}.get(d, d)


def decode_group_tile(heads, kvheads, dq, dv):
    """Query heads per workgroup; must match decode_group_tile() in decode_kernel.hip."""
    group = heads // kvheads
    per = (_tile_dim(dq) + _tile_dim(dv)) // 16
    gmax = 8 if per == 16 else 1
    while gmax < 4 and 2 * gmax * per <= 64:
        gmax *= 2
    tiles = -(-group // gmax)
    gt = 1
    while -(-group // gt) > tiles:
        gt *= 2
    return gt


def decode_workgroups_per_token(heads, kvheads, dq, dv):
    """Workgroups per (request, split): KV heads x ceil(group / GT)."""
    return kvheads * -(-(heads // kvheads) // decode_group_tile(heads, kvheads, dq, dv))


def decode_attention(q, k, v, *, cu_seqlens_q, cu_seqlens_k=None, seqused_k=None,
                     max_seqlen_k, block_table=None, softmax_scale=None, out=None,
                     leftpad_k=None, num_splits=0, s_aux=None, q_descale=None,
                     k_descale=None, v_descale=None, window_size=(-1, -1), softcap=0.,
                     alibi_slopes=None):
    """Attend one query per nonempty request, returning output and natural LSE.

    The caller supplies valid GPU sequence metadata with cu_seqlens_q
    differences in {0, 1}.  K/V are packed or paged, head dimensions lie in
    1..512.  FP8 descales, sinks, left windows and softcap run in the kernel.
    ALiBi slopes ([Hq] or [B, Hq]) add -slope |k_len - 1 - key| in the kernel.
    Public validation belongs to interface._run and the attention dispatcher.
    """
    tokens, heads, dq = q.shape
    kvheads, dv = k.shape[-2], v.shape[-1]
    batch = cu_seqlens_q.numel() - 1
    if tokens > batch:
        raise ValueError("decode accepts at most one query per request")
    out_dtype = torch.float16 if q.dtype == torch.float8_e4m3fn else q.dtype
    if out is None:
        out = torch.empty((tokens, heads, dv), dtype=out_dtype, device=q.device)
    lse = torch.empty((heads, tokens), dtype=torch.float32, device=q.device)
    if not tokens:
        return out, lse
    window_size = tuple(window_size)
    effective_max = min(max_seqlen_k, window_size[0] + 1) if window_size[0] >= 0 else max_seqlen_k
    keep = []
    args = build_args(q, k, v, out, lse, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                      seqused_k=seqused_k, max_seqlen_q=1, max_seqlen_k=max_seqlen_k,
                      block_table=block_table, softmax_scale=softmax_scale, causal=False,
                      window_size=window_size, alibi_slopes=alibi_slopes, softcap=softcap, s_aux=s_aux,
                      q_descale=q_descale, k_descale=k_descale, v_descale=v_descale,
                      mask_mod=None, aux_tensors=None, leftpad_k=leftpad_k, keep=keep)
    if _lib.supported("fa_decode_supported", args):
        groups = decode_workgroups_per_token(heads, kvheads, dq, dv)
        splits, span = split_plan(batch, groups, effective_max, num_splits)
        args.num_splits, args.split_span = splits, span
        if splits > 1:
            partial = torch.empty((batch, heads, splits, dv), dtype=torch.float32, device=q.device)
            partial_lse = torch.empty((batch, heads, splits), dtype=torch.float32, device=q.device)
            keep += [partial, partial_lse]
            args.partial_out, args.partial_lse = partial.data_ptr(), partial_lse.data_ptr()
        _lib.call("fa_decode_fwd", args, q.device)
        return out, lse
    # Dtype/dimension/stride combinations outside the decode kernel run the
    # generic kernel with the reference's split rule (_decode.py:63-64).
    splits = num_splits or max(1, min(32, (effective_max + 255) // 256))
    if splits > 1:
        partial = torch.empty((splits, tokens, heads, dv), device=q.device, dtype=torch.float32)
        partial_lse = torch.empty((splits, heads, tokens), device=q.device, dtype=torch.float32)
        keep += [partial, partial_lse]
        args.partial_out, args.partial_lse = partial.data_ptr(), partial_lse.data_ptr()
    args.num_splits = splits
    args.max_seqlen_q = 1
    _lib.call("fa_attn_fwd", args, q.device)
    return out, lse
