"""Attention dispatch onto the gfx950 kernels; no host request loop, no dense
score tensor, no read of device values.

Counterpart of flash_attn_mps/_attention.py:88-238.  The route depends only on
shapes, dtypes, strides, feature flags and the caller's maximum lengths:

1. one query per request, not deterministic, no mask -> split-KV decode
   (``_decode.decode_attention``; _attention.py:134-147, which also keeps
   ALiBi off that route);
2. bf16/fp16 with the feature set compiled into the MFMA prefill kernel
   (including per-request causality, and ALiBi without softcap, windows,
   per-request causality or FP8 K/V) -> fa_prefill_fwd (the reference's `fast` route, _attention.py:149-158);
   in a batch of several requests, the single-query ones go to the split-KV
   decode kernel first and fa_prefill_fwd skips them
   (FA_FLAG_SKIP_SINGLE_QUERY);
3. everything else -> fa_attn_fwd, the generic kernel, with the reference's
   split rule: deterministic -> 1, else num_splits, else
   min(32, ceil(max_k / 256)) when the row is decode-like or d > 256
   (_attention.py:159-161).
"""
import torch

from . import _lib

_TYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float8_e4m3fn)


def _i32(t, device, keep):
    if t is None:
        return None
    t = t.to(device=device, dtype=torch.int32)
    keep.append(t)
    return t


def _f32(t, device, keep):
    if t is None:
        return None
    t = t.to(device=device, dtype=torch.float32)
    keep.append(t)
    return t


def build_args(q, k, v, out, lse, *, cu_seqlens_q, cu_seqlens_k, seqused_k, max_seqlen_q,
               max_seqlen_k, block_table, softmax_scale, causal, window_size, alibi_slopes,
               softcap, s_aux, q_descale, k_descale, v_descale, mask_mod, aux_tensors,
               leftpad_k, keep):
    """Fill the fa_attn_args struct; `keep` collects converted temporaries."""
    dev = q.device
    a = _lib.AttnArgs()
    a.q, a.k, a.v, a.out, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
    a.q_dtype, a.k_dtype, a.v_dtype = (_lib.DTYPE_CODE[t.dtype] for t in (q, k, v))
    a.out_dtype = _lib.DTYPE_CODE[out.dtype]
    a.total_q, a.heads_q, a.head_dim_qk = q.shape
    a.heads_k, a.head_dim_v = k.shape[-2], v.shape[-1]
    a.batch = cu_seqlens_q.numel() - 1
    a.page_size = k.shape[1] if k.ndim == 4 else 0
    a.max_seqlen_q, a.max_seqlen_k = max_seqlen_q, max_seqlen_k
    a.q_stride[:] = q.stride()
    a.k_stride[:] = k.stride() if k.ndim == 4 else (0, *k.stride())
    a.v_stride[:] = v.stride() if v.ndim == 4 else (0, *v.stride())
    a.out_stride[:] = out.stride()
    a.lse_stride[:] = lse.stride()
    cq = _i32(cu_seqlens_q, dev, keep)
    a.cu_seqlens_q, a.cu_q_stride = cq.data_ptr(), cq.stride(0)
    ck = _i32(cu_seqlens_k, dev, keep)
    if ck is not None:
        a.cu_seqlens_k, a.cu_k_stride = ck.data_ptr(), ck.stride(0)
    used = _i32(seqused_k, dev, keep)
    if used is not None:
        a.seqused_k, a.used_k_stride = used.data_ptr(), used.stride(0)
    table = _i32(block_table, dev, keep)
    if table is not None:
        a.block_table = table.data_ptr()
        a.bt_stride[:] = table.stride()
    left = _i32(leftpad_k, dev, keep)
    if left is not None:
        a.leftpad_k, a.leftpad_stride = left.data_ptr(), left.stride(0)
    if isinstance(causal, torch.Tensor):
        flags = causal.to(device=dev, dtype=torch.bool)
        keep.append(flags)
        a.causal_by_batch, a.causal_stride = flags.data_ptr(), flags.stride(0)
        a.causal = 0
    else:
        a.causal = int(bool(causal))
    a.window_left, a.window_right = int(window_size[0]), int(window_size[1])
    kind = getattr(mask_mod, "kind", 0) if mask_mod is not None else 0
    a.mask_kind = kind
    a.mask_window = int(getattr(mask_mod, "sliding_window_left", -1)) if mask_mod is not None else -1
    a.mask_clamp = int(bool(getattr(mask_mod, "clamp_prefix_to_window", False))) if mask_mod is not None else 0
    if kind == 1:
        ranges = _i32(aux_tensors[0], dev, keep)
        a.mask_ranges = ranges.data_ptr()
        a.ranges_stride[:] = ranges.stride()
    elif kind == 2:
        prefix = _i32(aux_tensors[0], dev, keep)
        width = _i32(aux_tensors[1], dev, keep)
        a.mask_prefix, a.prefix_stride = prefix.data_ptr(), prefix.stride(0)
        a.mask_window_len = width.data_ptr()
    a.softmax_scale = float(softmax_scale if softmax_scale is not None else q.shape[-1] ** -0.5)
    a.softcap = float(softcap)
    alibi = _f32(alibi_slopes, dev, keep)
    if alibi is not None:
        a.alibi = alibi.data_ptr()
        a.alibi_stride[:] = (0, alibi.stride(0)) if alibi.ndim == 1 else alibi.stride()
    sinks = _f32(s_aux, dev, keep)
    if sinks is not None:
        a.sinks, a.sink_stride = sinks.data_ptr(), sinks.stride(0)
    for name, t in (("q_descale", q_descale), ("k_descale", k_descale), ("v_descale", v_descale)):
        t = _f32(t, dev, keep)
        if t is not None:
            setattr(a, name, t.data_ptr())
            getattr(a, name + "_stride")[:] = t.stride()
    a.num_splits, a.split_span = 1, 0
    return a


def _fast_candidate(q, k, v, out, num_splits, deterministic, causal, window_size, alibi_slopes,
                    s_aux, q_descale, k_descale, v_descale, mask_mod, leftpad_k):
    """Feature gate of the MFMA prefill route (kernel support is asked separately)."""
    return (not deterministic and num_splits in (0, 1)
            and q.dtype == out.dtype and q.dtype in (torch.float16, torch.bfloat16)
            and k.dtype == v.dtype and k.dtype in (q.dtype, torch.float8_e4m3fn)
            and mask_mod is None and leftpad_k is None)


def _decode_rows(args, batch, heads, kvheads, dq, dv, max_seqlen_k, device, keep):
    """Launch the split-KV decode kernel on the single-query requests of a
    mixed batch (it skips every other request); True if it ran."""
    if not _lib.supported("fa_decode_supported", args):
        return False
    from ._decode import decode_workgroups_per_token, split_plan
    groups = decode_workgroups_per_token(heads, kvheads, dq, dv)
    splits, span = split_plan(batch, groups, max_seqlen_k, 0)
    args.num_splits, args.split_span = splits, span
    if splits > 1:
        partial = torch.empty((batch, heads, splits, dv), dtype=torch.float32, device=device)
        partial_lse = torch.empty((batch, heads, splits), dtype=torch.float32, device=device)
        keep += [partial, partial_lse]
        args.partial_out, args.partial_lse = partial.data_ptr(), partial_lse.data_ptr()
    _lib.call("fa_decode_fwd", args, device)
    args.num_splits, args.split_span = 1, 0
    args.partial_out = args.partial_lse = None
    return True


def attention(q, k, v, *, cu_seqlens_q, cu_seqlens_k=None, seqused_k=None, max_seqlen_q,
              max_seqlen_k, block_table=None, softmax_scale=None, causal=False,
              window_size=(-1, -1), alibi_slopes=None, softcap=0., s_aux=None, q_descale=None,
              k_descale=None, v_descale=None, out=None, num_splits=0, mask_mod=None,
              aux_tensors=None, leftpad_k=None, deterministic=False):
    """Return packed output and natural-log LSE in ``[heads, total_q]`` order.

    All sequence metadata is consumed by the GPU.  Dispatch depends only on
    shapes and the caller's existing maximum lengths, never tensor values.
    """
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError("q, k and v must be on the same GPU (HIP) device")
    if q.ndim != 3 or k.ndim not in (3, 4) or v.ndim != k.ndim:
        raise ValueError("q must be packed 3-D; k/v must be packed 3-D or paged 4-D")
    if any(t.dtype not in _TYPES for t in (q, k, v)):
        raise TypeError("attention supports FP16, BF16, FP32 and FP8 E4M3FN")
    tokens, heads, dq = q.shape
    kh, dv = k.shape[-2], v.shape[-1]
    if not (1 <= dq <= 512 and 1 <= dv <= 512):
        raise ValueError("query/key and value head dimensions must be in 1..512")
    if k.shape[-1] != dq or v.shape[:-1] != k.shape[:-1]:
        raise ValueError("key/value shapes must agree except for their last dimension")
    if heads < 1 or kh < 1 or heads % kh:
        raise ValueError("query heads must be a positive multiple of KV heads")
    if (k.ndim == 4) != (block_table is not None):
        raise ValueError("paged 4-D KV requires block_table; packed 3-D KV does not")
    if cu_seqlens_k is None and seqused_k is None:
        raise ValueError("cu_seqlens_k or seqused_k is required")
    if num_splits < 0:
        raise ValueError("num_splits must be nonnegative")
    default_dtype = torch.float16 if q.dtype == torch.float8_e4m3fn else q.dtype
    if out is None:
        out = torch.empty((tokens, heads, dv), dtype=default_dtype, device=q.device)
    elif tuple(out.shape) != (tokens, heads, dv) or out.device != q.device:
        raise ValueError("out must have shape [total_q, query_heads, value_dim] on the GPU")
    if out.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("out must have FP16, BF16 or FP32 dtype")
    if tokens == 0:
        return out, torch.empty((heads, 0), device=q.device, dtype=torch.float32)
    if max_seqlen_q <= 0 or max_seqlen_k < 0:
        raise ValueError("nonempty q requires positive max_seqlen_q and nonnegative max_seqlen_k")
    batch = cu_seqlens_q.numel() - 1
    if batch < 1:
        raise ValueError("cu_seqlens_q must contain at least two offsets")
    if max_seqlen_q == 1 and not deterministic and mask_mod is None:
        # A single right-aligned query has no future keys, whatever `causal` says.
        from ._decode import decode_attention
        return decode_attention(
            q, k, v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
            seqused_k=seqused_k, max_seqlen_k=max_seqlen_k, block_table=block_table,
            softmax_scale=softmax_scale, out=out, leftpad_k=leftpad_k, num_splits=num_splits,
            s_aux=s_aux, q_descale=q_descale, k_descale=k_descale, v_descale=v_descale,
            window_size=window_size, softcap=softcap, alibi_slopes=alibi_slopes,
        )
    lse = torch.empty((heads, tokens), device=q.device, dtype=torch.float32)
    keep = []
    args = build_args(q, k, v, out, lse, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                      seqused_k=seqused_k, max_seqlen_q=max_seqlen_q, max_seqlen_k=max_seqlen_k,
                      block_table=block_table, softmax_scale=softmax_scale, causal=causal,
                      window_size=window_size, alibi_slopes=alibi_slopes, softcap=softcap,
                      s_aux=s_aux, q_descale=q_descale, k_descale=k_descale, v_descale=v_descale,
                      mask_mod=mask_mod, aux_tensors=aux_tensors, leftpad_k=leftpad_k, keep=keep)
    if (_fast_candidate(q, k, v, out, num_splits, deterministic, causal, window_size, alibi_slopes,
                        s_aux, q_descale, k_descale, v_descale, mask_mod, leftpad_k)
            and _lib.supported("fa_prefill_supported", args)):
        # Mixed batches (chunked prefill + decode): single-query requests run
        # on the split-KV decode kernel and the MFMA kernel skips them, since a
        # 128-row query tile would spend one workgroup per head on each.  When
        # the same offsets describe queries and keys (packed self-attention), a
        # single-query request has a single key, so the MFMA kernel keeps it
        # and no decode pass is launched.
        self_attention = cu_seqlens_k is cu_seqlens_q and seqused_k is None and block_table is None
        if (batch > 1 and not self_attention
                and _decode_rows(args, batch, heads, kh, dq, dv, max_seqlen_k, q.device, keep)):
            args.flags |= _lib.FLAG_SKIP_SINGLE_QUERY
        _lib.call("fa_prefill_fwd", args, q.device)
        return out, lse
    vector = deterministic or max_seqlen_q == 1 or max(dq, dv) > 256
    splits = 1 if deterministic else num_splits or (
        min(32, max(1, (max_seqlen_k + 255) // 256)) if vector else 1)
    if splits > 1:
        partial = torch.empty((splits, tokens, heads, dv), device=q.device, dtype=torch.float32)
        partial_lse = torch.empty((splits, heads, tokens), device=q.device, dtype=torch.float32)
        keep += [partial, partial_lse]
        args.partial_out, args.partial_lse = partial.data_ptr(), partial_lse.data_ptr()
    args.num_splits = splits
    _lib.call("fa_attn_fwd", args, q.device)
    return out, lse
