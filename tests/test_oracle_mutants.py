"""Planted mistakes in copies of the CPU attention oracle (CPU only).

Each mutant is oracle/attention.py with one plausible mistake substituted
into its source text (a dropped term, a wrong sign, index or alignment, a
swapped operand), compiled into a throw-away namespace.  Every mutant must
fail at least one check of oracle_pins.ALL_CHECKS; the real oracle passes
them all (test_oracle_attention.py).  Nothing here touches a GPU.
"""
from pathlib import Path

import pytest

import oracle_pins

SOURCE = (Path(__file__).resolve().parents[1] / "oracle" / "attention.py").read_text()

MUTANTS = {
    "top-left causal alignment": ("qpos = (length - qlen + idx)[:, None]", "qpos = idx[:, None]"),
    "softcap without the inner division": ("torch.tanh(scores / softcap) * softcap", "torch.tanh(scores) * softcap"),
    "sink dropped from the denominator": ("logits = torch.cat((scores, sink), dim=-1)", "logits = scores"),
    "ALiBi sign flipped": ("scores = scores - slopes[:, None, None]", "scores = scores + slopes[:, None, None]"),
    "left window off by one": ("keep = keep & (diff <= window[0])", "keep = keep & (diff < window[0])"),
    "right window sign": ("keep = keep & (-diff <= window[1])", "keep = keep & (diff <= window[1])"),
    "GQA head map interleaved": ("kv_of_head = torch.arange(heads) // group", "kv_of_head = torch.arange(heads) % hkv"),
    "LSE in log2 units": ("lse[:, start + idx] = row_lse", "lse[:, start + idx] = row_lse * 1.4426950408889634"),
    "page and offset swapped": ("key, value = k[phys, pos % page], v[phys, pos % page]",
                                "key, value = k[phys, pos // page], v[phys, pos // page]"),
    "paged leftpad ignored": ("pos = left[b] + torch.arange(length)", "pos = torch.arange(length)"),
    "packed cu_seqlens_k ignored": ("base = (cuk[b] if cuk is not None else 0) + left[b]", "base = left[b]"),
    "default scale from Dv": ("scale = dq ** -0.5 if scale is None", "scale = dv ** -0.5 if scale is None"),
    "v descale dropped": ("value = value * s[:, None, None]", "value = value"),
    "q descale applied to v": ("query = query * s[:, None, None]", "value = value * s[:, None, None]"),
    "rswa prefix inclusive": ("(kpos < prefix_len)", "(kpos <= prefix_len)"),
    "mm_prefix window inclusive": ("keep &= diff < width", "keep &= diff <= width"),
    "causal_by_batch ignored": ("is_causal = causal_by_batch[b] if causal_by_batch is not None",
                                "is_causal = causal_by_batch[0] if causal_by_batch is not None"),
    "fully masked rows become NaN": ("probs = torch.exp(scores - row_lse.unsqueeze(-1)).nan_to_num(0.0)",
                                     "probs = torch.exp(scores - row_lse.unsqueeze(-1))"),
    "softcap output mis-scaled": ("        if softcap:\n            scores = torch.tanh(scores / softcap) * softcap\n",
                                  "        if softcap:\n            scores = torch.tanh(scores / softcap) * softcap * 1.0001\n"),
    "scale applied twice": ("scores = torch.matmul(query, key.transpose(-2, -1)) * scale",
                            "scores = torch.matmul(query, key.transpose(-2, -1)) * scale * scale"),
}


def _mutant(old, new):
    assert SOURCE.count(old) == 1, f"mutation site not unique: {old!r}"
    namespace = {"__name__": "oracle_attention_mutant"}
    exec(compile(SOURCE.replace(old, new), "oracle_attention_mutant", "exec"), namespace)
    return namespace["attention"]


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_is_caught(name):
    attn = _mutant(*MUTANTS[name])
    caught = []
    for check in oracle_pins.ALL_CHECKS:
        try:
            check(attn)
        except Exception as exc:  # an assertion or a crash both expose the mutant
            caught.append(f"{check.__name__}: {type(exc).__name__}")
    assert caught, f"no pin check catches the planted mistake '{name}'"
