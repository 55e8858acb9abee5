"""Model-level parity: the paged-KV serving engine of benchmarks/validate_engine.py on this package's
kernels vs an fp32 PyTorch attention over the same caches (counterpart of the reference's
benchmarks/validate_nanovllm.py:18-200).  A 2-layer Qwen3-shaped decoder with seeded random weights
keeps the run short; the attention shapes (16/8 heads x 128) are the real ones.  Each case must give
finite logits, per-step KL <= 1e-3 nats, greedy agreement wherever the choice is numerically decided,
and exercise its engine feature (prefix-cache hits, chunked prefill, preemption)."""
import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "flash-attn-mps_amd" / "benchmarks"))
import validate_engine as ve  # noqa: E402

pytestmark = pytest.mark.gpu

CFG = ve.ModelConfig(layers=2, hidden=512, intermediate=1024, vocab=8192)


@pytest.fixture(scope="module")
def weights():
    return ve.init_weights(CFG, torch.device("cuda", 0))


@pytest.mark.parametrize("name", [c[0] for c in ve.cases()])
def test_engine_case(device, weights, name):
    settings, batches = next((s, b) for n, s, b in ve.cases() if n == name)
    with torch.inference_mode():
        ref, trace = ve.run_case(CFG, weights, settings, batches, ve.reference_attention, device)
        native, _ = ve.run_case(CFG, weights, settings, batches, ve.native_attention, device, expected=trace)
    assert native["errors"], "no sampler calls"
    assert ve.check(name, ref, native, batches) == []


@pytest.mark.parametrize("name", ["normal", "preemption"])
def test_engine_case_graph_captured_decode(device, weights, name):
    """The decode step captured in HIP graphs (per batch size, padded rows) meets the same bar."""
    settings, batches = next((s, b) for n, s, b in ve.cases() if n == name)
    with torch.inference_mode():
        ref, trace = ve.run_case(CFG, weights, settings, batches, ve.reference_attention, device)
        native, _ = ve.run_case(CFG, weights, settings, batches, ve.native_attention, device, expected=trace,
                                graphs=True)
    assert ve.check(name, ref, native, batches) == []
