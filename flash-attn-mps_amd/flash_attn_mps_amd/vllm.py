"""vLLM FLASH_ATTN / FLASH_ATTN_DIFFKV tensor contract on MI355X.

Counterpart of flash_attn_mps/vllm.py (vLLM 0.29.0's argument order):
per-request ("dynamic") causality, the multimodal-prefix and rolling-window
masks, FP8 descales ``[B, Hkv]`` (broadcast views allowed), attention sinks
(``s_aux``), caller-owned ``out``, split-KV and LSE merging for cascade /
decode-context-parallel attention.  It registers no vLLM platform and moves
no data between GPUs: ``merge_attn_states`` is the local combine step of
whatever transport the engine uses.
"""
from ._problem import MaskSpec, Problem, reject_training


def mm_prefix_mask(sliding_window_left=None, clamp_prefix_to_window=False):
    """Multimodal-prefix mask: causal (optionally windowed) attention plus, per
    query row, the key range ``aux_tensors[0][row]`` = [lo, hi] (lo < 0: none).

    Pass ``aux_tensors=[ranges int32 [T, 2], cu_seqlens_q int32 [B+1]]``.
    ``clamp_prefix_to_window`` also applies the window to the prefix range.
    """
    window = -1 if sliding_window_left is None else int(sliding_window_left)
    if window < 1 and window != -1:
        raise ValueError(f"sliding_window_left={sliding_window_left}: use a positive width or None")
    if clamp_prefix_to_window and window == -1:
        raise ValueError("clamp_prefix_to_window needs a sliding_window_left")
    return MaskSpec(1, window, bool(clamp_prefix_to_window))


def rswa_mask():
    """Rolling sliding-window mask: causal, keys before ``prefix[b]`` always
    visible, later keys only within ``window[0]`` positions.

    Pass ``aux_tensors=[prefix int32 [B], window int32 [1]]``.
    """
    return MaskSpec(2)


def get_scheduler_metadata(*args, **kwargs):
    """vLLM asks for CUDA scheduler metadata; the gfx950 kernels plan on their own."""
    return None


# vLLM arguments outside the FLASH_ATTN contract, and why each is refused.
_UNSUPPORTED = (
    ("q_v", lambda x: x is not None, "q_v (MLA) is not part of the FLASH_ATTN contract"),
    ("cp_world_size", lambda x: x != 1, "context parallelism (cp_world_size) is not supported"),
    ("cp_rank", lambda x: x != 0, "context parallelism (cp_rank) is not supported"),
    ("cp_tot_seqused_k", lambda x: x is not None, "context parallelism (cp_tot_seqused_k) is not supported"),
    ("block_sparse_tensors", lambda x: x is not None, "block-sparse attention is a separate backend"),
    ("output_scale", lambda x: x is not None, "fused output quantization (output_scale) is not supported"),
    ("aux_tensor_leading_dims", lambda x: x is not None, "custom auxiliary tensor layouts are not supported"),
)


def flash_attn_varlen_func(
    q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k,
    cu_seqlens_k=None, seqused_k=None, q_v=None, dropout_p=0.0,
    softmax_scale=None, causal=False, window_size=None, softcap=0.0,
    alibi_slopes=None, deterministic=False, return_attn_probs=False,
    block_table=None, return_softmax_lse=False, out=None, scheduler_metadata=None,
    q_descale=None, k_descale=None, v_descale=None, num_splits=0,
    output_scale=None, fa_version=2, s_aux=None, cp_world_size=1,
    cp_rank=0, cp_tot_seqused_k=None, mask_mod=None, block_sparse_tensors=None,
    aux_tensors=None, aux_tensor_leading_dims=None, dynamic_causal=None,
):
    """vLLM's attention call: packed or paged K/V, vLLM argument order.

    ``fa_version`` (2, 3 or 4) and ``scheduler_metadata`` are accepted as
    hints and change nothing.  ``dynamic_causal`` (bool [B]) overrides
    ``causal`` per request.  ``num_splits=1`` (or ``deterministic``) gives
    every query row a fixed reduction order whatever else is in the batch.
    Paged K/V requires ``seqused_k``.
    """
    reject_training(dropout_p, return_attn_probs, (q, k, v))
    if fa_version not in (2, 3, 4):
        raise ValueError(f"fa_version={fa_version}: expected 2, 3 or 4")
    given = dict(q_v=q_v, cp_world_size=cp_world_size, cp_rank=cp_rank, cp_tot_seqused_k=cp_tot_seqused_k,
                 block_sparse_tensors=block_sparse_tensors, output_scale=output_scale,
                 aux_tensor_leading_dims=aux_tensor_leading_dims)
    for name, refused, reason in _UNSUPPORTED:
        if refused(given[name]):
            raise NotImplementedError(reason)
    if block_table is not None:
        if k.ndim != 4 or k.shape[1] % 16:
            raise ValueError(f"a paged cache needs page sizes that are multiples of 16; got k {tuple(k.shape)}")
        if seqused_k is None:
            raise ValueError("paged K/V in the vLLM contract needs seqused_k")
    fixed_order = deterministic or num_splits == 1
    problem = Problem(q, k, v, cu_seqlens_q, max_seqlen_q, max_seqlen_k, cu_k=cu_seqlens_k,
                      used_k=seqused_k, table=block_table, scale=softmax_scale,
                      causal=causal if dynamic_causal is None else dynamic_causal,
                      window=(-1, -1) if window_size is None else tuple(window_size), softcap=softcap,
                      alibi=alibi_slopes, sinks=s_aux, q_descale=q_descale, k_descale=k_descale,
                      v_descale=v_descale, mask=mask_mod,
                      mask_aux=None if aux_tensors is None else tuple(aux_tensors), out=out,
                      splits=1 if deterministic else num_splits, deterministic=fixed_order)
    from ._attention import solve
    result, lse = solve(problem.validate())
    return (result, lse) if return_softmax_lse else result


def merge_attn_states(output, prefix_output, prefix_lse, suffix_output, suffix_lse, output_lse=None):
    """Combine two attention states over disjoint key sets (cascade or DCP).

    States are [T, H, D] with natural-log LSE [H, T]; writes ``output`` (and
    ``output_lse`` if given), which may alias the inputs.
    """
    from ._merge import merge_attn_states as merge
    merge(output, prefix_output, prefix_lse, suffix_output, suffix_lse, out_lse=output_lse)
