"""Route a validated Problem onto the gfx950 kernels.

Counterpart of flash_attn_mps/_attention.py:88-238.  The route depends only on
shapes, dtypes, strides, feature flags and the caller's maximum lengths --
never on device values, so a call never synchronises and can be captured in
a HIP graph:

1. one query per request, not deterministic, no vLLM mask -> split-KV decode
   (`_decode.decode`; the reference's decode route, _attention.py:134-147);
2. inputs whose feature set the MFMA prefill kernel compiles
   (fa_prefill_supported) -> fa_prefill_fwd (the reference's `fast` route,
   _attention.py:149-158, which this kernel widens to windows, sinks, FP8
   K/V, E4M3 queries, ALiBi and per-request causality); in a batch of
   several requests the single-query ones go to the decode kernel first and
   fa_prefill_fwd skips them (FA_FLAG_SKIP_SINGLE_QUERY);
3. everything else -> fa_attn_fwd, the generic kernel, with the reference's
   split rule: deterministic -> 1, else num_splits, else min(32, ceil(max_k /
   256)) when the row is decode-like or d > 256 (_attention.py:159-161).

Deterministic calls (vLLM's num_splits=1, the reference's fixed
batch-invariant path, docs/contracts.md:76-79) take route 2 for every
request, single-query ones included, or route 3 with one split.  Either
kernel computes a row from its own request alone, in a fixed order: query
blocks and key tiles are aligned to the request's first query and key, the
kernel variant depends only on dtypes, head dims and feature flags, and a
key tile that a row cannot see adds exact zeros to its sums.  So a request's
rows are bit-identical whatever else is in the batch.
"""
import torch

from . import _lib


def _as(t, dtype, keep):
    """`t` as a device tensor of `dtype` (kept alive until the launch is enqueued)."""
    if t is None:
        return None
    if t.dtype != dtype:
        t = t.to(dtype)
    keep.append(t)
    return t


def build_args(p, out, lse, max_q=None):
    """The fa_attn_args struct of problem `p` writing `out` / `lse`."""
    keep = p.keep
    a = _lib.AttnArgs()
    a.q, a.k, a.v = p.q.data_ptr(), p.k.data_ptr(), p.v.data_ptr()
    a.out, a.lse = out.data_ptr(), lse.data_ptr()
    a.q_dtype, a.k_dtype, a.v_dtype = (_lib.DTYPE_CODE[t.dtype] for t in (p.q, p.k, p.v))
    a.out_dtype = _lib.DTYPE_CODE[out.dtype]
    a.total_q, a.heads_q, a.head_dim_qk = p.q.shape
    a.heads_k, a.head_dim_v = p.kv_heads, p.dim_v
    a.batch = p.batch
    a.page_size = p.k.shape[1] if p.paged else 0
    a.max_seqlen_q = p.max_q if max_q is None else max_q
    a.max_seqlen_k = p.max_k
    a.q_stride[:] = p.q.stride()
    a.k_stride[:] = p.k.stride() if p.paged else (0, *p.k.stride())
    a.v_stride[:] = p.v.stride() if p.paged else (0, *p.v.stride())
    a.out_stride[:] = out.stride()
    a.lse_stride[:] = lse.stride()
    i32 = torch.int32
    cu_q = _as(p.cu_q, i32, keep)
    a.cu_seqlens_q, a.cu_q_stride = cu_q.data_ptr(), cu_q.stride(0)
    for tensor, ptr_field, stride_field in ((p.cu_k, "cu_seqlens_k", "cu_k_stride"),
                                            (p.used_k, "seqused_k", "used_k_stride"),
                                            (p.leftpad, "leftpad_k", "leftpad_stride")):
        t = _as(tensor, i32, keep)
        if t is not None:
            setattr(a, ptr_field, t.data_ptr())
            setattr(a, stride_field, t.stride(0))
    table = _as(p.table, i32, keep)
    if table is not None:
        a.block_table = table.data_ptr()
        a.bt_stride[:] = table.stride()
    if torch.is_tensor(p.causal):
        flags = _as(p.causal, torch.bool, keep)
        a.causal_by_batch, a.causal_stride, a.causal = flags.data_ptr(), flags.stride(0), 0
    else:
        a.causal = int(bool(p.causal))
    a.window_left, a.window_right = (int(w) for w in p.window)
    if p.mask is not None:
        a.mask_kind = p.mask.kind
        a.mask_window = int(p.mask.sliding_window_left)
        a.mask_clamp = int(bool(p.mask.clamp_prefix_to_window))
        first, second = (_as(t, i32, keep) for t in p.mask_aux)
        if p.mask.kind == 1:
            a.mask_ranges = first.data_ptr()
            a.ranges_stride[:] = first.stride()
        else:
            a.mask_prefix, a.prefix_stride = first.data_ptr(), first.stride(0)
            a.mask_window_len = second.data_ptr()
    else:
        a.mask_kind, a.mask_window, a.mask_clamp = 0, -1, 0
    a.softmax_scale = float(p.dim_qk ** -0.5 if p.scale is None else p.scale)
    a.softcap = float(p.softcap)
    f32 = torch.float32
    alibi = _as(p.alibi, f32, keep)
    if alibi is not None:
        a.alibi = alibi.data_ptr()
        a.alibi_stride[:] = (0, alibi.stride(0)) if alibi.ndim == 1 else alibi.stride()
    sinks = _as(p.sinks, f32, keep)
    if sinks is not None:
        a.sinks, a.sink_stride = sinks.data_ptr(), sinks.stride(0)
    for name in ("q_descale", "k_descale", "v_descale"):
        t = _as(getattr(p, name), f32, keep)
        if t is not None:
            setattr(a, name, t.data_ptr())
            getattr(a, name + "_stride")[:] = t.stride()
    a.num_splits, a.split_span = 1, 0
    return a


def _fits_prefill(p, out):
    """Features the MFMA route takes at all (the kernel is asked about the rest,
    vLLM mask kinds and left padding included): 16-bit queries over same-type
    or E4M3 K/V with output in the query's type, or E4M3 queries over E4M3 K/V
    with fp16/bf16 output (S on the FP8 MFMA).  The kernel never splits a row,
    so deterministic calls qualify."""
    if p.splits not in (0, 1):
        return False
    fp8 = torch.float8_e4m3fn
    if p.k.dtype != p.v.dtype:
        return False
    if p.q.dtype == fp8:
        return p.k.dtype == fp8 and out.dtype in (torch.float16, torch.bfloat16)
    return (p.q.dtype in (torch.float16, torch.bfloat16) and out.dtype == p.q.dtype
            and p.k.dtype in (p.q.dtype, fp8))


def _partials(p, a, shape_out, shape_lse):
    """fp32 split workspace for the generic kernel or the decode kernel."""
    po = torch.empty(shape_out, dtype=torch.float32, device=p.device)
    pl = torch.empty(shape_lse, dtype=torch.float32, device=p.device)
    p.keep += [po, pl]
    a.partial_out, a.partial_lse = po.data_ptr(), pl.data_ptr()


_SIDE = {}

# Below this many K/V bytes (an upper bound of what the decode pass of a
# mixed batch reads: every request at the longest visible length) the decode
# pass follows the prefill on the caller's stream: it takes a few µs of GPU
# time, less than the host time of the cross-stream fork and join (an event
# record and a stream wait each way, ~30 µs per call measured on short calls).
_SIDE_STREAM_MIN_BYTES = 64 << 20


def _side_stream(device):
    """A second stream per device (default priority) for the decode rows of a
    mixed batch, with the two events that fork and join it (reused: a stream
    wait takes the event's most recent record)."""
    index = torch.device(device).index
    side = _SIDE.get(index)
    if side is None:
        side = _SIDE[index] = (torch.cuda.Stream(device), torch.cuda.Event(), torch.cuda.Event())
    return side


def _mixed_batch(p, a, fixed_order=False):
    """A batch of several requests with single-query ones among them: the
    decode kernel takes the single-query requests (it skips the others) and
    fa_prefill_fwd the rest (FA_FLAG_SKIP_SINGLE_QUERY).  The two kernels
    write disjoint rows, so they run concurrently: the prefill is enqueued
    first on the caller's stream and the decode on a side stream that starts
    after the caller's earlier work; the caller's stream then waits for it.
    The memory-bound decode fills the CUs the compute-bound prefill leaves.
    Small calls (under _SIDE_STREAM_MIN_BYTES of K/V) run both on the
    caller's stream, one after the other.
    Returns False (nothing launched) when the decode kernel cannot take the
    single-query rows.  With `fixed_order` the decode runs one split per
    request, so each single-query row is reduced in an order of its own
    request only (the batch-invariant route)."""
    dec = _lib.AttnArgs.from_buffer_copy(a)
    dec.max_seqlen_q = 1   # the decode kernel takes the one-row requests only
    if not _lib.supported("fa_decode_supported", dec):
        return False
    from ._decode import decode_workgroups, split_plan
    groups = decode_workgroups(p, 1)
    splits, span = split_plan(p.batch, groups, p.max_k, 1 if fixed_order else 0)
    dec.num_splits, dec.split_span = splits, span
    if splits > 1:
        _partials(p, dec, (p.batch, splits, p.heads, p.dim_v), (p.batch, p.heads, splits))
    a.flags |= _lib.FLAG_SKIP_SINGLE_QUERY
    kv_bytes = p.batch * p.visible_max * p.kv_heads * (p.dim_qk + p.dim_v) * p.k.element_size()
    if kv_bytes < _SIDE_STREAM_MIN_BYTES:
        _lib.call("fa_prefill_fwd", a, p.device)
        _lib.call("fa_decode_fwd", dec, p.device)
        return True
    main = torch.cuda.current_stream(p.device)
    side, fork, join = _side_stream(p.device)
    fork.record(main)
    side.wait_event(fork)
    _lib.call("fa_prefill_fwd", a, p.device)
    with torch.cuda.stream(side):
        _lib.call("fa_decode_fwd", dec, p.device)
    join.record(side)
    main.wait_event(join)
    return True


def _fixed_order_decode(p, out):
    """A fixed-order (deterministic / vLLM num_splits=1) call whose requests
    all hold one query row: the decode kernel with one split per request, on
    paged K/V, exactly when a batch holding these requests next to longer
    ones would route them to it (_mixed_batch), so a request's result does
    not depend on its neighbours.  Packed K/V keep the MFMA prefill: the
    matrix-core decode aligns its key stages to storage rows, which move
    with a request's place in the batch.  None when this route does not
    apply (nothing launched)."""
    if not p.paged or not _fits_prefill(p, out):
        return None
    lse = torch.empty((p.heads, p.tokens), device=p.device, dtype=torch.float32)
    a = build_args(p, out, lse)
    if not (_lib.supported("fa_prefill_supported", a) and _lib.supported("fa_decode_supported", a)):
        return None
    from ._decode import decode
    return decode(p, out, splits=1)


def solve(p):
    """Run a validated Problem: returns (out [T, Hq, Dv], natural-log lse [Hq, T])."""
    out = p.out
    if out is None:
        out = torch.empty((p.tokens, p.heads, p.dim_v), dtype=p.output_dtype, device=p.device)
    if p.tokens == 0:
        return out, torch.empty((p.heads, 0), device=p.device, dtype=torch.float32)
    if p.max_q <= 0:
        raise ValueError("nonempty queries need max_seqlen_q >= 1")
    if p.batch < 1:
        raise ValueError("cu_seqlens_q needs at least two offsets")
    if p.max_q == 1 and not p.deterministic and p.mask is None:
        from ._decode import decode
        return decode(p, out)
    if p.max_q == 1 and p.deterministic and p.mask is None:
        done = _fixed_order_decode(p, out)
        if done is not None:
            return done
    if p.max_q > 1 and not p.deterministic and p.mask is None:
        # A few query rows per request (speculative / multi-token decode):
        # the matrix-core decode with (head, row) columns when it takes them.
        from ._decode import decode_rows
        done = decode_rows(p, out)
        if done is not None:
            return done
    lse = torch.empty((p.heads, p.tokens), device=p.device, dtype=torch.float32)
    a = build_args(p, out, lse)
    if _fits_prefill(p, out) and _lib.supported("fa_prefill_supported", a):
        # In a mixed chunked-prefill + decode batch the single-query requests
        # take the decode kernel: a 128-row MFMA query tile per head would be
        # almost empty for them.  Packed self-attention (queries and keys on
        # the same offsets) gives a single-query request a single key, so the
        # MFMA kernel keeps it and no decode pass runs.  Deterministic calls
        # keep every request in this kernel (the decode kernel's split count
        # follows the batch).
        self_attention = p.cu_k is p.cu_q and p.used_k is None and not p.paged
        mixed = p.batch > 1 and not self_attention and (not p.deterministic or p.paged)
        if not (mixed and _mixed_batch(p, a, fixed_order=p.deterministic)):
            _lib.call("fa_prefill_fwd", a, p.device)
        return out, lse
    per_row = p.deterministic or p.max_q == 1 or max(p.dim_qk, p.dim_v) > 256
    if p.deterministic:
        splits = 1
    else:
        splits = p.splits or (min(32, max(1, -(-p.max_k // 256))) if per_row else 1)
    if splits > 1:
        _partials(p, a, (splits, p.tokens, p.heads, p.dim_v), (splits, p.heads, p.tokens))
    a.num_splits = splits
    _lib.call("fa_attn_fwd", a, p.device)
    return out, lse
