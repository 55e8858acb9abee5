"""Log-sum-exp merging of independently computed attention states on gfx950.

Host side of fa_merge_pair / fa_merge_partials; mirrors
flash_attn_mps/_merge.py:20-57 (shape/dtype checks, in-place aliasing,
optional output LSE).
"""
import torch

from . import _lib
from ._cache import _gpu


def merge_attn_states(out, left_out, left_lse, right_out, right_lse, out_lse=None):
    """Write the LSE-weighted merge to ``out``; LSE uses natural logarithms.

    Outputs are [tokens, heads, dim], LSE tensors are FP32 [heads, tokens].
    An empty state has LSE=-inf; merging two empty states yields zero and -inf.
    ``out`` and ``out_lse`` may alias the corresponding input states.
    """
    _gpu(out, left_out, left_lse, right_out, right_lse, out_lse)
    if out.ndim != 3 or left_out.shape != out.shape or right_out.shape != out.shape:
        raise ValueError("output states must have matching [tokens, heads, dim] shapes")
    if left_out.dtype != out.dtype or right_out.dtype != out.dtype:
        raise TypeError("output state dtypes must match")
    if out.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("output states must be float16, bfloat16 or float32")
    expected = (out.shape[1], out.shape[0])
    for lse in (left_lse, right_lse, out_lse):
        if lse is not None and (tuple(lse.shape) != expected or lse.dtype != torch.float32):
            raise ValueError("LSE tensors must be float32 [heads, tokens]")
    if not out.numel():
        return
    a = _lib.MergePairArgs()
    a.out, a.a, a.b = out.data_ptr(), left_out.data_ptr(), right_out.data_ptr()
    a.a_lse, a.b_lse, a.out_lse = left_lse.data_ptr(), right_lse.data_ptr(), _lib.ptr(out_lse)
    a.dtype = _lib.DTYPE_CODE[out.dtype]
    a.tokens, a.heads, a.dim = out.shape
    a.out_stride[:], a.a_stride[:], a.b_stride[:] = out.stride(), left_out.stride(), right_out.stride()
    a.a_lse_stride[:], a.b_lse_stride[:] = left_lse.stride(), right_lse.stride()
    a.out_lse_stride[:] = out_lse.stride() if out_lse is not None else (0, 0)
    _lib.call("fa_merge_pair", a, out.device)


def _merge_partials(partial_out, partial_lse):
    """Merge [splits, tokens, heads, dim] and [splits, heads, tokens] states."""
    _gpu(partial_out, partial_lse)
    if partial_out.ndim != 4 or partial_lse.shape != (partial_out.shape[0], partial_out.shape[2],
                                                      partial_out.shape[1]):
        raise ValueError("partial states require [splits,tokens,heads,dim] and [splits,heads,tokens]")
    if partial_lse.dtype != torch.float32:
        raise TypeError("partial LSE must be float32")
    if partial_out.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("partial states must be float16, bfloat16 or float32")
    splits, tokens, heads, dim = partial_out.shape
    output = torch.empty((tokens, heads, dim), dtype=partial_out.dtype, device=partial_out.device)
    lse = torch.empty((heads, tokens), dtype=torch.float32, device=partial_out.device)
    if tokens and heads:
        a = _lib.MergePartialsArgs()
        a.partial, a.partial_lse = partial_out.data_ptr(), partial_lse.data_ptr()
        a.out, a.lse = output.data_ptr(), lse.data_ptr()
        a.partial_dtype = a.out_dtype = _lib.DTYPE_CODE[partial_out.dtype]
        a.splits, a.tokens, a.heads, a.dim = splits, tokens, heads, dim
        a.partial_stride[:] = partial_out.stride()
        a.partial_lse_stride[:] = partial_lse.stride()
        a.out_stride[:] = output.stride()
        a.lse_stride[:] = lse.stride()
        _lib.call("fa_merge_partials", a, partial_out.device)
    return output, lse
