"""The complete-call comparison against a per-request ROCm SDPA serving loop
(flash-attn-mps_amd/benchmarks/compare_sdpa.py, after the reference's release
gate, benchmarks/bench_attention.py:24-108 and docs/validation.md:15).

Every case of its matrix (prefill B1/B4 x 2K/4K, decode B1/4/16 x 4K/8K
contexts, the short cases) runs the native path -- store_kvcache of the new
tokens, then varlen prefill or paged decode -- and is held to the CPU oracle
at the parity bar (fp16 2e-3, LSE 1e-4 where returned).  The script itself
then runs end to end in its --quick mode on one case, as a user would.
"""
import json
import math
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from harness import assert_parity, oracle_attention

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "flash-attn-mps_amd" / "benchmarks"))
import compare_sdpa  # noqa: E402

pytestmark = pytest.mark.gpu

CASES = {c[0]: c[1:] for c in compare_sdpa.cases()}


@pytest.mark.parametrize("name", list(CASES))
def test_native_path_matches_the_oracle(device, name):
    batch, qlen, klen, prefill, _ = CASES[name]
    q, k, v, kc, vc, ctx = compare_sdpa.make_case(batch, qlen, klen, prefill, device)
    with torch.inference_mode():
        got = compare_sdpa.native_path(q, k, v, kc, vc, ctx)
    torch.cuda.synchronize()
    page = compare_sdpa.PAGE
    worst = 0.0
    for b in range(batch):
        rows = slice(b * qlen, (b + 1) * qlen)
        if ctx.block_tables is None:      # self-attention over the new tokens themselves
            ref, _ = oracle_attention(q[rows], k[rows], v[rows], torch.tensor([0, qlen], dtype=torch.int32),
                                      torch.tensor([0, qlen], dtype=torch.int32), scale=compare_sdpa.SCALE,
                                      causal=True, dtype=torch.float32, chunk=1024)
        else:                             # the request's pages, after the slot writes
            pages = ctx.block_tables[b, :math.ceil(klen / page)].long()
            table = torch.arange(pages.numel(), dtype=torch.int32).reshape(1, -1)
            ref, _ = oracle_attention(q[rows], kc[pages].cpu(), vc[pages].cpu(),
                                      torch.tensor([0, qlen], dtype=torch.int32), used_k=torch.tensor([klen]),
                                      block_table=table, scale=compare_sdpa.SCALE, causal=True,
                                      dtype=torch.float32, chunk=1024)
        worst = max(worst, assert_parity(got[rows], None, ref, None, torch.float16, what=f"{name} request {b}")[0])
    print(f"{name}: max |native - oracle| {worst:.2e}")


def test_comparison_script_runs_end_to_end(tmp_path):
    out = tmp_path / "compare.json"
    run = subprocess.run([sys.executable, str(ROOT / "flash-attn-mps_amd" / "benchmarks" / "compare_sdpa.py"),
                          "--quick", "--case", "decode-b4-k4096", "--output", str(out)],
                         capture_output=True, text=True, timeout=100)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-2000:]
    report = json.loads(out.read_text())
    case = report["cases"][0]
    assert case["name"] == "decode-b4-k4096" and case["max_abs_error"] <= 3e-3
    assert case["median_speedup"] > 0 and case["graph"]["speedup"] > 0
