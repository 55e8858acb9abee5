"""Log-sum-exp merging of attention states on gfx950 (host side of
fa_merge_pair / fa_merge_partials; counterpart of flash_attn_mps/_merge.py:20-57).

A state is an output [T, H, D] with its natural-log LSE [H, T] over some key
set.  Merging states over disjoint key sets gives the state over their union:
weights exp(lse_i - lse), lse = log(sum exp(lse_i)).  An empty state has
LSE -inf and weight 0 (its payload is never read); +inf takes all the weight.
"""
import torch

from . import _lib
from ._problem import Want, on_gpu

_STATE_TYPES = (torch.float16, torch.bfloat16, torch.float32)


def _on_one_gpu(tensors):
    present = [t for t in tensors if t is not None]
    for t in present:
        if not on_gpu(t):
            raise ValueError(f"merge inputs must be GPU tensors; got one on {t.device}")
    return present[0].device


def merge_attn_states(out, left_out, left_lse, right_out, right_lse, out_lse=None):
    """out = merge(left, right); out / out_lse may alias the left or right state.

    Outputs share one shape [T, H, D] and dtype (fp16/bf16/fp32); LSE tensors
    are fp32 [H, T] with any strides.
    """
    device = _on_one_gpu((out, left_out, left_lse, right_out, right_lse, out_lse))
    if out.ndim != 3:
        raise ValueError(f"merged states are [tokens, heads, dim]; out has shape {tuple(out.shape)}")
    tokens, heads, dim = out.shape
    for name, t in (("left output", left_out), ("right output", right_out)):
        Want(name, (tokens, heads, dim)).check(t, device)
        if t.dtype != out.dtype:
            raise TypeError(f"{name} is {t.dtype} but out is {out.dtype}; states share one dtype")
    if out.dtype not in _STATE_TYPES:
        raise TypeError(f"states are float16, bfloat16 or float32; got {out.dtype}")
    for name, t in (("left lse", left_lse), ("right lse", right_lse), ("out lse", out_lse)):
        Want(name, (heads, tokens), (torch.float32,)).check(t, device)
    if out.numel() == 0:
        return
    a = _lib.MergePairArgs()
    a.out, a.a, a.b = out.data_ptr(), left_out.data_ptr(), right_out.data_ptr()
    a.a_lse, a.b_lse, a.out_lse = left_lse.data_ptr(), right_lse.data_ptr(), _lib.ptr(out_lse)
    a.dtype = _lib.DTYPE_CODE[out.dtype]
    a.tokens, a.heads, a.dim = tokens, heads, dim
    a.out_stride[:], a.a_stride[:], a.b_stride[:] = out.stride(), left_out.stride(), right_out.stride()
    a.a_lse_stride[:], a.b_lse_stride[:] = left_lse.stride(), right_lse.stride()
    a.out_lse_stride[:] = out_lse.stride() if out_lse is not None else (0, 0)
    _lib.call("fa_merge_pair", a, device)


def merge_partials(partial_out, partial_lse):
    """Merge S states at once: partial_out [S, T, H, D], partial_lse fp32 [S, H, T]
    (any strides) -> fresh (out [T, H, D] of partial_out's dtype, lse [H, T])."""
    device = _on_one_gpu((partial_out, partial_lse))
    if partial_out.ndim != 4:
        raise ValueError(f"partial outputs are [splits, tokens, heads, dim]; got {tuple(partial_out.shape)}")
    splits, tokens, heads, dim = partial_out.shape
    if tuple(partial_lse.shape) != (splits, heads, tokens):
        raise ValueError(f"partial lse has shape {tuple(partial_lse.shape)}; expected {(splits, heads, tokens)}")
    if partial_lse.dtype != torch.float32:
        raise TypeError(f"partial lse must be float32; got {partial_lse.dtype}")
    if partial_out.dtype not in _STATE_TYPES:
        raise TypeError(f"partial outputs are float16, bfloat16 or float32; got {partial_out.dtype}")
    out = torch.empty((tokens, heads, dim), dtype=partial_out.dtype, device=device)
    lse = torch.empty((heads, tokens), dtype=torch.float32, device=device)
    if tokens and heads:
        a = _lib.MergePartialsArgs()
        a.partial, a.partial_lse = partial_out.data_ptr(), partial_lse.data_ptr()
        a.out, a.lse = out.data_ptr(), lse.data_ptr()
        a.partial_dtype = a.out_dtype = _lib.DTYPE_CODE[partial_out.dtype]
        a.splits, a.tokens, a.heads, a.dim = splits, tokens, heads, dim
        a.partial_stride[:] = partial_out.stride()
        a.partial_lse_stride[:] = partial_lse.stride()
        a.out_stride[:] = out.stride()
        a.lse_stride[:] = lse.stride()
        _lib.call("fa_merge_partials", a, device)
    return out, lse
