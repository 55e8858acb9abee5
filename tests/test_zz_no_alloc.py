"""fa_decode_fwd_noalloc: split-KV decode whose partials live in the library's
own per-GPU device array, checked against fa_decode_fwd with caller-allocated
partials on the same arguments.

The same split plan runs the same kernels, so those results are bit-identical;
a plan that the array forces to fewer splits is held to the parity bar instead
(max |out| difference <= 1e-2 for bf16, LSE <= 1e-4).  Calls run back to back
with shrinking inputs, since the array keeps the previous call's contents.
"""
import ctypes

import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd._decode import decode_workgroups, split_plan, workgroups_per_token
from harness import kernel_args, problem

pytestmark = pytest.mark.gpu

PAGE = 16


def _paged_case(device, *, batch, heads, kvheads, dim, max_ctx, pool_pages, kv_dtype, seed,
                window=(-1, -1), softcap=0.0, sinks=False):
    """Decode arguments over a shared page pool: block-table rows index a pool
    of `pool_pages` pages at random (rows may repeat pages), so large batches
    need little memory."""
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(1, max_ctx + 1, (batch,), generator=g, dtype=torch.int32)
    cols = -(-max_ctx // PAGE)
    table = torch.randint(0, pool_pages, (batch, cols), generator=g, dtype=torch.int32)
    q = torch.randn(batch, heads, dim, generator=g).to(torch.bfloat16)
    kc = torch.randn(pool_pages, PAGE, kvheads, dim, generator=g)
    vc = torch.randn(pool_pages, PAGE, kvheads, dim, generator=g)
    if kv_dtype == torch.float8_e4m3fn:
        kc, vc = (x.clamp(-448, 448).to(kv_dtype) for x in (kc, vc))
    else:
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
    t = dict(q=q.to(device), k=kc.to(device), v=vc.to(device),
             cu_q=torch.arange(batch + 1, dtype=torch.int32).to(device),
             used=lengths.to(device), table=table.to(device))
    if kv_dtype == torch.float8_e4m3fn:
        t["k_descale"] = (torch.rand(batch, kvheads, generator=g) * 0.09 + 0.01).to(device)
        t["v_descale"] = (torch.rand(batch, kvheads, generator=g) * 0.09 + 0.01).to(device)
    if sinks:
        t["s_aux"] = torch.randn(heads, generator=g).to(device)
    t.update(max_ctx=max_ctx, window=window, softcap=softcap)
    return t


def _args(t, out, lse, keep):
    return kernel_args(t["q"], t["k"], t["v"], out, lse, keep=keep, cu_seqlens_q=t["cu_q"], seqused_k=t["used"],
                       max_seqlen_q=1, max_seqlen_k=t["max_ctx"], block_table=t["table"], window_size=t["window"],
                       softcap=t["softcap"], s_aux=t.get("s_aux"), k_descale=t.get("k_descale"),
                       v_descale=t.get("v_descale"))


def _outputs(t):
    batch, heads, dim = t["q"].shape
    out = torch.full((batch, heads, dim), float("nan"), dtype=torch.bfloat16, device=t["q"].device)
    lse = torch.full((heads, batch), float("nan"), dtype=torch.float32, device=t["q"].device)
    return out, lse


def _python_plan(t):
    batch, heads, dim = t["q"].shape
    p = problem(t["q"], t["k"], t["v"], cu_seqlens_q=t["cu_q"], seqused_k=t["used"], max_seqlen_q=1,
                max_seqlen_k=t["max_ctx"], block_table=t["table"])
    groups = decode_workgroups(p)
    wl = t["window"][0]
    visible = min(t["max_ctx"], wl + 1) if wl >= 0 else t["max_ctx"]
    return split_plan(batch, groups, visible, 0)


def _decode_fwd(t):
    """fa_decode_fwd with partial buffers allocated here (the Python path's plan)."""
    keep = []
    out, lse = _outputs(t)
    a = _args(t, out, lse, keep)
    splits, span = _python_plan(t)
    a.num_splits, a.split_span = splits, span
    batch, heads, dim = t["q"].shape
    if splits > 1:
        po = torch.empty(batch, splits, heads, dim, dtype=torch.float32, device=out.device)
        pl = torch.empty(batch, heads, splits, dtype=torch.float32, device=out.device)
        keep += [po, pl]
        a.partial_out, a.partial_lse = po.data_ptr(), pl.data_ptr()
    _lib.call("fa_decode_fwd", a, out.device)
    torch.cuda.synchronize()
    return out, lse, splits


def _noalloc(t, num_splits=0, span=0):
    keep = []
    out, lse = _outputs(t)
    a = _args(t, out, lse, keep)
    a.num_splits, a.split_span = num_splits, span
    _lib.call("fa_decode_fwd_noalloc", a, out.device)
    torch.cuda.synchronize()
    return out, lse


def _partial_bytes(t, splits):
    batch, heads, dim = t["q"].shape
    return batch * heads * splits * (dim + 1) * 4


CASES = {
    # Llama-3-8B-like bf16 (config 3's heads and dims), then smaller inputs.
    "bf16_32x8_d128": dict(batch=48, heads=32, kvheads=8, dim=128, max_ctx=12000, pool_pages=900,
                           kv_dtype=torch.bfloat16),
    "bf16_16x2_d64_sinks": dict(batch=9, heads=16, kvheads=2, dim=64, max_ctx=3000, pool_pages=200,
                                kv_dtype=torch.bfloat16, sinks=True),
    # Gemma-2-like FP8 cache with descales, softcap and a left window (config 4's features).
    "fp8_16x8_d256_window_softcap": dict(batch=20, heads=16, kvheads=8, dim=256, max_ctx=6000,
                                         pool_pages=400, kv_dtype=torch.float8_e4m3fn,
                                         window=(4095, 0), softcap=50.0),
    # GQA groups of 16 and 5: the matrix-core decode (bf16, and FP8 with descales).
    "bf16_64x4_d128_gqa": dict(batch=24, heads=64, kvheads=4, dim=128, max_ctx=9000, pool_pages=700,
                               kv_dtype=torch.bfloat16, sinks=True),
    "fp8_40x8_d128_gqa_softcap": dict(batch=16, heads=40, kvheads=8, dim=128, max_ctx=5000, pool_pages=400,
                                      kv_dtype=torch.float8_e4m3fn, softcap=30.0),
}


def test_noalloc_matches_decode_fwd_on_consecutive_shrinking_calls(device):
    names = list(CASES)
    for seed, name in enumerate(names):
        t = _paged_case(device, seed=100 + seed, **CASES[name])
        ref_out, ref_lse, splits = _decode_fwd(t)
        assert splits > 1, f"{name}: the case should exercise the partials"
        assert _partial_bytes(t, splits) <= _lib.DECODE_SCRATCH_BYTES
        out, lse = _noalloc(t)
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), name
        assert torch.equal(lse, ref_lse), name
        # The caller's own plan (the same one) takes the same route.
        out2, lse2 = _noalloc(t, *_python_plan(t))
        assert torch.equal(out2.view(torch.int16), ref_out.view(torch.int16)), name
        assert torch.equal(lse2, ref_lse), name


def test_noalloc_second_call_with_smaller_input(device):
    big = _paged_case(device, seed=7, **CASES["bf16_32x8_d128"])
    small = _paged_case(device, seed=8, **dict(CASES["bf16_32x8_d128"], batch=5, max_ctx=2500))
    for t in (big, small):
        ref_out, ref_lse, _ = _decode_fwd(t)
        out, lse = _noalloc(t)
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(lse, ref_lse)


def test_noalloc_reduces_its_plan_to_fit_the_array(device):
    # 512 requests x 64 query heads: the Python plan's partials (8 splits,
    # ~135 MB) exceed the 32 MiB array, so the library runs fewer splits.
    t = _paged_case(device, seed=11, batch=512, heads=64, kvheads=8, dim=128, max_ctx=16384,
                    pool_pages=512, kv_dtype=torch.bfloat16)
    ref_out, ref_lse, splits = _decode_fwd(t)
    assert _partial_bytes(t, splits) > _lib.DECODE_SCRATCH_BYTES
    out, lse = _noalloc(t)
    out_err = (out.double() - ref_out.double()).abs().max().item()
    lse_err = (lse.double() - ref_lse.double()).abs().max().item()
    assert out_err <= 1e-2 and lse_err <= 1e-4, (out_err, lse_err)


def test_noalloc_rejects_plans_that_do_not_fit_and_caller_buffers(device):
    t = _paged_case(device, seed=12, **CASES["bf16_32x8_d128"])
    splits = 64
    assert _partial_bytes(t, splits) > _lib.DECODE_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="limit"):
        _noalloc(t, splits, -(-t["max_ctx"] // splits))
    keep = []
    out, lse = _outputs(t)
    a = _args(t, out, lse, keep)
    a.num_splits, a.split_span = 2, t["max_ctx"]
    a.partial_out = a.partial_lse = out.data_ptr()
    rc = _lib.load().fa_decode_fwd_noalloc(ctypes.byref(a), _lib.stream_of(device))
    assert rc == 1 and b"library-owned" in _lib.load().fa_last_error()


def test_noalloc_multi_row_decode_matches_decode_rows(device):
    """Speculative-decode rows (1-4 per request, causal): the library's plan
    equals the Python layer's, so fa_decode_fwd_noalloc and decode_rows (with
    caller-allocated partials) give bit-identical results; then a smaller call."""
    from flash_attn_mps_amd._decode import decode_rows
    for seed, (batch, max_ctx) in enumerate([(24, 9000), (3, 700)]):
        t = _paged_case(device, seed=40 + seed, batch=batch, heads=32, kvheads=8, dim=128, max_ctx=max_ctx,
                        pool_pages=700, kv_dtype=torch.bfloat16, sinks=True)
        g = torch.Generator().manual_seed(50 + seed)
        q_lens = torch.randint(1, 5, (batch,), generator=g).tolist()
        q_lens[0] = 4
        cu_q = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0)), dtype=torch.int32, device=device)
        q = torch.randn(sum(q_lens), 32, 128, generator=g).to(torch.bfloat16).to(device)
        kw = dict(cu_seqlens_q=cu_q, seqused_k=t["used"], max_seqlen_q=4, max_seqlen_k=max_ctx,
                  block_table=t["table"], s_aux=t["s_aux"], causal=True)
        p = problem(q, t["k"], t["v"], **kw).validate()
        ref_out, ref_lse = decode_rows(p, torch.full_like(q, float("nan")))
        splits, _ = split_plan(batch, workgroups_per_token(32, 8, 128, 128, True, 4), max_ctx, 0)
        assert splits > 1, "the case should exercise the partials"
        keep = []
        out, lse = torch.full_like(q, float("nan")), torch.full_like(ref_lse, float("nan"))
        a = kernel_args(q, t["k"], t["v"], out, lse, keep=keep, **kw)
        a.num_splits, a.split_span = 0, 0
        _lib.call("fa_decode_fwd_noalloc", a, device)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(lse, ref_lse)
