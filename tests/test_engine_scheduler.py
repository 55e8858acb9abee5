"""CPU checks of the serving engine in benchmarks/validate_engine.py (block manager, chunked
prefill, prefix caching, preemption) with a stand-in model, so the GPU parity test exercises an
engine whose scheduling is known to terminate and to hit each feature."""
import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "flash-attn-mps_amd" / "benchmarks"))
import validate_engine as ve  # noqa: E402


class CountingModel:
    """Logits that prefer (last token + position) % vocab; records every step's shapes."""

    def __init__(self, vocab=64):
        self.vocab, self.steps = vocab, []

    def forward(self, ids, positions, ctx, last_index):
        self.steps.append((ctx.is_prefill, list(ctx.q_lens), list(ctx.k_lens), ctx.slot_mapping.tolist(),
                           ctx.block_tables.tolist()))
        logits = torch.zeros(len(last_index), self.vocab)
        for r, i in enumerate(last_index.tolist()):
            logits[r, (int(ids[i]) + int(positions[i])) % self.vocab] = 1.0
        return logits


def greedy(logits, seqs):
    return logits.argmax(-1).tolist()


def run(settings, batches):
    model = CountingModel()
    eng = ve.Engine(model, settings["num_blocks"], settings["max_num_seqs"], settings["max_num_batched_tokens"], "cpu")
    outs = [eng.generate(p, n, greedy, first_sid=10 * k) for k, (p, n) in enumerate(batches)]
    return eng, model, outs


@pytest.mark.parametrize("name", [c[0] for c in ve.cases()])
def test_engine_cases_complete(name):
    settings, batches = next((s, b) for n, s, b in ve.cases() if n == name)
    eng, model, outs = run(settings, batches)
    for (prompts, n), o in zip(batches, outs):
        assert [len(x) for x in o] == [n] * len(prompts)
    assert sorted(eng.bm.free) == list(range(settings["num_blocks"]))          # everything released
    c = eng.counters
    if name == "shared-prefix":
        assert c["prefix_hits"] == 2
        # the second batch computes only the unshared suffix of each prompt
        second = [s for s in model.steps if s[0]][-1]
        assert second[1] == [9, 13] and second[2] == [521, 525]
    if name == "chunked-prefill":
        chunks = [s[1][0] for s in model.steps if s[0]]
        assert chunks == [128] * 6 + [777 - 6 * 128]
    if name == "preemption":
        assert c["preemptions"] == 1 and c["prefill_steps"] == 2


def test_slots_follow_block_tables():
    settings, batches = next((s, b) for n, s, b in ve.cases() if n == "cross-page")
    eng, model, _ = run(settings, batches)
    for is_prefill, q_lens, k_lens, slots, tables in model.steps:
        start = 0
        for b, (ql, kl) in enumerate(zip(q_lens, k_lens)):
            for j, pos in enumerate(range(kl - ql, kl)):
                assert slots[start + j] == tables[b][pos // ve.PAGE] * ve.PAGE + pos % ve.PAGE
            start += ql


def test_outputs_do_not_depend_on_schedule():
    """The stand-in model is position-exact, so chunking, prefix reuse and preemption must not change
    the generated tokens."""
    prompt = list(range(5, 5 + 300))
    plain, _, (a,) = run(dict(max_num_seqs=4, max_num_batched_tokens=1024, num_blocks=16), [([prompt], 12)])
    chunked, _, (b,) = run(dict(max_num_seqs=4, max_num_batched_tokens=64, num_blocks=16), [([prompt], 12)])
    assert a == b
