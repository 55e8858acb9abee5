"""Test harness: keyword-built attention problems, the CPU oracle, and the parity bar.

* `problem(...)` / `attention(...)` / `decode_attention(...)` / `kernel_args(...)`
  build a `Problem` from keyword arguments and run it through the package's
  router, the decode path, or just the C-struct builder.
* `oracle_attention(...)` is the CPU restatement under /oracle, computed in
  float64 (float32 and row chunks for full-size configurations).
* `assert_parity(...)` is the acceptance bar of this build (north star):
  max |out - oracle| <= 2e-3 for fp16 outputs, <= 1e-2 for bf16, <= 1e-4 for
  fp32; max |lse - oracle| <= 1e-4.  Rows whose LSE is -inf in the oracle must
  be -inf in the result too.
"""
import torch

from flash_attn_mps_amd._attention import build_args, solve
from flash_attn_mps_amd._decode import decode
from flash_attn_mps_amd._problem import Problem
from oracle.attention import attention as _oracle

OUT_BAR = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-4}
LSE_BAR = 1e-4

_KEYWORDS = dict(cu_seqlens_k="cu_k", seqused_k="used_k", block_table="table", leftpad_k="leftpad",
                 softmax_scale="scale", window_size="window", alibi_slopes="alibi", s_aux="sinks",
                 mask_mod="mask", aux_tensors="mask_aux", num_splits="splits")


def problem(q, k, v, *, cu_seqlens_q, max_seqlen_q, max_seqlen_k, **kw):
    """A Problem from the keyword names of the public API."""
    fields = {_KEYWORDS.get(name, name): value for name, value in kw.items()}
    if "window" in fields:
        fields["window"] = tuple(fields["window"])
    if fields.get("mask_aux") is not None:
        fields["mask_aux"] = tuple(fields["mask_aux"])
    return Problem(q, k, v, cu_seqlens_q, max_seqlen_q, max_seqlen_k, **fields)


def attention(q, k, v, **kw):
    """Route through the package (decode / MFMA prefill / generic), after validation."""
    return solve(problem(q, k, v, **kw).validate())


def decode_attention(q, k, v, *, max_seqlen_k, out=None, **kw):
    """The single-query path (split-KV decode kernel, or the generic kernel it falls back to)."""
    p = problem(q, k, v, max_seqlen_q=1, max_seqlen_k=max_seqlen_k, out=out, **kw).validate()
    if out is None:
        out = torch.empty((p.tokens, p.heads, p.dim_v), dtype=p.output_dtype, device=p.device)
    if p.tokens == 0:
        return out, torch.empty((p.heads, 0), dtype=torch.float32, device=p.device)
    return decode(p, out)


def kernel_args(q, k, v, out, lse, *, keep, **kw):
    """The fa_attn_args struct of a call (its temporaries appended to `keep`)."""
    p = problem(q, k, v, **kw)
    keep.append(p)
    return build_args(p, out, lse)


def oracle_attention(q, k, v, cu_q, cu_k=None, used_k=None, dtype=torch.float64, chunk=None, **kw):
    """The CPU oracle; with `chunk`, query rows are evaluated `chunk` at a time
    (attention rows are independent, so this is exact and bounds memory)."""
    if chunk is None:
        return _oracle(q, k, v, cu_q, cu_k=cu_k, used_k=used_k, dtype=dtype, **kw)
    total = q.shape[0]
    out = torch.zeros(total, q.shape[1], v.shape[-1], dtype=dtype)
    lse = torch.full((q.shape[1], total), -torch.inf, dtype=dtype)
    for start in range(0, total, chunk):
        rows = torch.arange(start, min(total, start + chunk))
        o, l = _oracle(q, k, v, cu_q, cu_k=cu_k, used_k=used_k, dtype=dtype, rows=rows, **kw)
        out[rows], lse[:, rows] = o[rows], l[:, rows]
    return out, lse


def max_err(actual, expected):
    """max |actual - expected| where equal infinities count as 0."""
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    if a.numel() == 0:
        return 0.0
    same = (a == e) | (torch.isnan(a) & torch.isnan(e))
    diff = torch.where(same, torch.zeros_like(a), (a - e).abs())
    return float(diff.nan_to_num(float("inf")).max())


def assert_parity(out, lse, ref, ref_lse, out_dtype=None, *, rows=None, out_bar=None, lse_bar=LSE_BAR, what=""):
    """Check (out, lse) against the oracle at the parity bar; returns the errors.

    lse is [Hq, T] (or any layout matching ref_lse); `rows` restricts the
    check to those packed query rows; out_bar defaults to the bar of out's
    dtype."""
    dtype = out_dtype or out.dtype
    if rows is not None:
        rows = torch.as_tensor(rows, dtype=torch.long)
        out, ref = out.detach().cpu()[rows], ref[rows]
        if lse is not None:
            lse, ref_lse = lse.detach().cpu()[:, rows], ref_lse[:, rows]
    bar = OUT_BAR[dtype] if out_bar is None else out_bar
    out_err = max_err(out, ref)
    assert out_err <= bar, f"{what} max |out - oracle| = {out_err:.3e} > {bar:.1e} ({dtype})"
    lse_err = None
    if lse is not None:
        lse_err = max_err(lse, ref_lse)
        assert lse_err <= lse_bar, f"{what} max |lse - oracle| = {lse_err:.3e} > {lse_bar:.1e}"
        empty = torch.isneginf(ref_lse.detach().cpu())
        assert torch.isneginf(lse.detach().cpu()[empty]).all(), f"{what} rows with no visible key must give -inf"
    return out_err, lse_err


def offsets(lengths, device=None):
    """int32 cumulative offsets [0, l0, l0+l1, ...]."""
    c = [0]
    for n in lengths:
        c.append(c[-1] + int(n))
    return torch.tensor(c, dtype=torch.int32, device=device)


def seeded(shape, seed, dtype, device, scale=1.0):
    """N(0, scale^2) drawn on the CPU from `seed`, cast to `dtype`, then moved:
    the GPU and the oracle see identical values."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * scale
    return x.to(dtype).to(device)
