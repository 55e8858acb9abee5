"""Complete-call comparison with a per-request PyTorch SDPA serving path on ROCm.

Mirrors the case matrix and method of the reference's release-gate benchmark
(benchmarks/bench_attention.py:24-70, 121-124, 140-166): each timed call
includes the slot writes of the new tokens, the metadata handling and the
attention itself.

* Baseline: the per-request loop a serving engine runs without a native
  varlen kernel — ``index_copy_`` slot writes, a gather of each request's
  pages, and ``torch.nn.functional.scaled_dot_product_attention`` with a
  lower-right causal bias and GQA.  SDPA is restricted to its fused flash /
  memory-efficient backends on ROCm.
* Native: ``store_kvcache`` + ``flash_attn_varlen_func`` (prefill) or
  ``flash_attn_with_kvcache`` (decode) of this package.

fp16, 16 query / 8 KV heads, head dim 128, 256-token pages, physical page
order a random permutation.  Every case is checked against the baseline
(atol 3e-3, rtol 1e-2, as the reference does) before it is timed; timing is
wall clock around each call plus a device synchronize, p50/p95 over
``--iterations``, ``--rounds`` rounds with alternating order.

Decode cases also time the native step captured in a HIP graph and replayed.

usage: python flash-attn-mps_amd/benchmarks/compare_sdpa.py --output result.json [--quick] [--case NAME]
"""
import argparse
import json
import math
import statistics
import sys
import time
from pathlib import Path
from types import SimpleNamespace

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel
from torch.nn.attention.bias import causal_lower_right

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import flash_attn_mps_amd as fa  # noqa: E402

HQ, HKV, D, PAGE = 16, 8, 128, 256
SCALE = D ** -0.5


def cases():
    rows = [(f"prefill-b{b}-s{s}", b, s, s, True, True) for b in (1, 4) for s in (2048, 4096)]
    rows += [(f"decode-b{b}-k{k}", b, 1, k, False, True) for b in (1, 4, 16) for k in (4096, 8192)]
    rows += [("short-prefill", 1, 128, 128, True, False), ("short-decode", 1, 1, 256, False, False),
             ("cached-prefill", 4, 64, 576, True, False)]
    return rows


def make_case(batch, qlen, klen, prefill, device):
    """Requests of qlen new tokens at the end of klen-token contexts."""
    gen = torch.Generator().manual_seed(123)
    pages = math.ceil(klen / PAGE)
    table_cpu = torch.randperm(batch * pages, generator=gen).reshape(batch, pages)
    q = torch.randn(batch * qlen, HQ, D, generator=gen).half().to(device)
    k = torch.randn(batch * qlen, HKV, D, generator=gen).half().to(device)
    v = torch.randn(batch * qlen, HKV, D, generator=gen).half().to(device)
    kc = torch.randn(batch * pages, PAGE, HKV, D, generator=gen).half().to(device)
    vc = torch.randn(batch * pages, PAGE, HKV, D, generator=gen).half().to(device)
    pos = torch.arange(klen - qlen, klen)
    slots = torch.cat([table_cpu[b, pos // PAGE] * PAGE + pos % PAGE for b in range(batch)])
    ctx = SimpleNamespace(
        is_prefill=prefill, max_q=qlen, max_k=klen,
        slot_mapping=slots.to(device=device, dtype=torch.int32),
        cu_seqlens_q=torch.arange(batch + 1, device=device, dtype=torch.int32) * qlen,
        cu_seqlens_k=torch.arange(batch + 1, device=device, dtype=torch.int32) * klen,
        context_lens=torch.full((batch,), klen, device=device, dtype=torch.int32),
        block_tables=table_cpu.to(device=device, dtype=torch.int32) if (not prefill or klen > qlen) else None,
        # host copies a serving engine keeps beside the device metadata
        q_offsets=[qlen * b for b in range(batch + 1)], k_lengths=[klen] * batch,
    )
    return q, k, v, kc, vc, ctx


_GQA = {"native": None}


def sdpa_gqa(query, key, value, qlen, klen):
    """SDPA with GQA; expands K/V heads when the fused backends reject enable_gqa."""
    bias = causal_lower_right(qlen, klen)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        if _GQA["native"] is not False:
            try:
                out = F.scaled_dot_product_attention(query, key, value, attn_mask=bias, scale=SCALE, enable_gqa=True)
                _GQA["native"] = True
                return out
            except RuntimeError:
                if _GQA["native"]:
                    raise
                _GQA["native"] = False
        rep = query.shape[1] // key.shape[1]
        return F.scaled_dot_product_attention(query, key.repeat_interleave(rep, dim=1),
                                              value.repeat_interleave(rep, dim=1), attn_mask=bias, scale=SCALE)


def sdpa_path(q, k, v, kc, vc, ctx):
    if kc.numel():
        slots = ctx.slot_mapping.long()
        kc.flatten(0, 1).index_copy_(0, slots, k)
        vc.flatten(0, 1).index_copy_(0, slots, v)
    offsets = ctx.q_offsets
    outs = []
    for i, length in enumerate(ctx.k_lengths):
        start, end = offsets[i], offsets[i + 1]
        query = q[start:end].transpose(0, 1).unsqueeze(0).contiguous()
        if ctx.block_tables is not None:
            blocks = ctx.block_tables[i, :math.ceil(length / PAGE)].long()
            key = kc[blocks].flatten(0, 1)[:length]
            value = vc[blocks].flatten(0, 1)[:length]
        else:
            key, value = k[start:end], v[start:end]
        key = key.transpose(0, 1).unsqueeze(0).contiguous()
        value = value.transpose(0, 1).unsqueeze(0).contiguous()
        outs.append(sdpa_gqa(query, key, value, end - start, length).squeeze(0).transpose(0, 1))
    return torch.cat(outs)


def native_path(q, k, v, kc, vc, ctx):
    fa.store_kvcache(k, v, kc, vc, ctx.slot_mapping)
    if ctx.is_prefill:
        key, value = (kc, vc) if ctx.block_tables is not None else (k, v)
        return fa.flash_attn_varlen_func(q, key, value, ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.max_q, ctx.max_k,
                                         softmax_scale=SCALE, causal=True, block_table=ctx.block_tables)
    return fa.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, cache_seqlens=ctx.context_lens,
                                      block_table=ctx.block_tables, softmax_scale=SCALE,
                                      causal=True).reshape_as(q)


def measure(fn, args, warmup, iterations):
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    samples = []
    for _ in range(iterations):
        t0 = time.perf_counter()
        fn(*args)
        torch.cuda.synchronize()
        samples.append((time.perf_counter() - t0) * 1e3)
    ordered = sorted(samples)
    return {"p50_ms": statistics.median(samples), "p95_ms": ordered[math.ceil(0.95 * len(ordered)) - 1]}


def graph_replay(args, opts):
    """Decode step (slot write + attention) captured once and replayed.

    The host layer reads no device values, so the captured call is the same
    work; replay removes the per-launch host overhead that dominates small
    batches.  The replay output must equal the eager output.
    """
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            native_path(*args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = native_path(*args)
    eager = native_path(*args)
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(captured, eager):
        raise AssertionError("graph replay differs from the eager call")
    eager_t = measure(native_path, args, opts.warmup, opts.iterations)
    graph_t = measure(graph.replay, (), opts.warmup, opts.iterations)
    return {"eager": eager_t, "replay": graph_t, "speedup": eager_t["p50_ms"] / graph_t["p50_ms"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--iterations", type=int, default=50)
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--case")
    ap.add_argument("--quick", action="store_true", help="5 iterations, 1 round, 2 warmup")
    opts = ap.parse_args()
    if not torch.cuda.is_available():
        sys.exit("compare_sdpa.py needs a GPU")
    if opts.quick:
        opts.iterations, opts.rounds, opts.warmup = 5, 1, 2
    device = torch.device("cuda", 0)
    todo = [c for c in cases() if opts.case in (None, c[0])]
    if not todo:
        sys.exit(f"unknown case {opts.case}")
    report = {"torch": torch.__version__, "device": torch.cuda.get_device_name(device), "dtype": "float16",
              "heads": [HQ, HKV], "head_dim": D, "page_size": PAGE, "iterations": opts.iterations,
              "rounds": opts.rounds, "warmup": opts.warmup,
              "baseline": "per-request torch SDPA (flash / mem-efficient backends) + index_copy_ slot writes",
              "cases": []}
    opts.output.parent.mkdir(parents=True, exist_ok=True)
    with torch.inference_mode():
        for name, batch, qlen, klen, prefill, gate in todo:
            args = make_case(batch, qlen, klen, prefill, device)
            t0 = time.perf_counter()
            actual = native_path(*args)
            torch.cuda.synchronize()
            first_ms = (time.perf_counter() - t0) * 1e3
            expected = sdpa_path(*args)
            torch.testing.assert_close(actual, expected, atol=3e-3, rtol=1e-2)
            row = {"name": name, "release_gate": gate, "first_call_ms": first_ms,
                   "max_abs_error": float((actual - expected).abs().max()), "rounds": []}
            del actual, expected
            for rnd in range(opts.rounds):
                order = [("sdpa", sdpa_path), ("native", native_path)]
                if rnd % 2:
                    order.reverse()
                times = {label: measure(fn, args, opts.warmup, opts.iterations) for label, fn in order}
                times["speedup"] = times["sdpa"]["p50_ms"] / times["native"]["p50_ms"]
                row["rounds"].append(times)
                print(name, rnd + 1, json.dumps(times), flush=True)
            row["median_speedup"] = statistics.median(r["speedup"] for r in row["rounds"])
            if not prefill:
                row["graph"] = graph_replay(args, opts)
                print(name, "graph", json.dumps(row["graph"]), flush=True)
            report["cases"].append(row)
            opts.output.write_text(json.dumps(report, indent=2) + "\n")
            del args
            torch.cuda.empty_cache()
    report["sdpa_enable_gqa"] = _GQA["native"]
    opts.output.write_text(json.dumps(report, indent=2) + "\n")


if __name__ == "__main__":
    main()
