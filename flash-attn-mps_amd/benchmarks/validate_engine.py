"""Model-level check: a paged-KV serving engine on this package's kernels vs an fp32 PyTorch attention.

Counterpart of the reference's nano-vLLM validation (benchmarks/validate_nanovllm.py:18-200), which
needs nano-vLLM and a local checkpoint.  Neither exists on an offline box, so this file carries its own
small engine and a Qwen3-0.6B-shaped decoder with seeded random weights:

* Engine: block manager over 256-token pages with prefix caching (hash chains over full blocks, kept
  after a sequence finishes), a scheduler with chunked prefill (`max_num_batched_tokens`) and
  preemption by recomputation when decode runs out of blocks.
* Model: Qwen3 layout (RMSNorm, per-head q/k RMSNorm, NeoX RoPE theta 1e6, GQA 16/8 x 128, SwiGLU),
  fp16 weights ~N(0, 0.02) and an untied fp32 lm_head ~N(0, 0.08), wide enough that the next-token
  distribution is peaked and greedy agreement means something.
* Attention backends, both over the same fp16 paged caches:
  - native: `store_kvcache` + `flash_attn_varlen_func` (prefill chunks and prefix-cached prefill,
    paged) + `flash_attn_with_kvcache` (decode) — the three entry points the reference patches into
    nano-vLLM (benchmarks/bench_nanovllm_optimization.py:57-61);
  - reference: `index_copy_` slot writes, a per-request gather of the pages and fp32 softmax
    attention with lower-right causality.

The reference run records logits and greedy tokens; the native run is teacher-forced with those
tokens and must give finite logits, per request and step KL(P_ref || P_native) <= 1e-3 nats at
temperature 1 (validate_nanovllm.py:18, 100-104) and the same greedy choices wherever the reference's
top-2 logit gap exceeds twice the row's largest logit difference (random weights make near-ties
likelier than a trained model does; they are reported, not failed).  Cases mirror the
reference's (validate_nanovllm.py:165-171): normal, cross-page, shared-prefix (prefix-cache hits),
chunked-prefill, preemption.

Every case also runs natively with the decode step captured in HIP graphs (one per batch size,
replayed with the step's inputs in static buffers) and must meet the same criteria.  With
--performance it also times greedy generation (batch 1 and 4, 1024-token prompts, 128 new tokens):
this package's kernels eager and graph-captured against per-request torch SDPA.

usage: python flash-attn-mps_amd/benchmarks/validate_engine.py --output report.json [--layers 28] [--case NAME]
       [--performance]
"""
import argparse
import itertools
import json
import math
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import flash_attn_mps_amd as fa  # noqa: E402

KL_LIMIT = 1e-3
PAGE = 256


@dataclass
class ModelConfig:
    layers: int = 28
    hidden: int = 1024
    intermediate: int = 3072
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    rope_theta: float = 1e6
    eps: float = 1e-6
    lm_head_std: float = 0.08
    seed: int = 0


def init_weights(cfg, device, dtype=torch.float16):
    g = torch.Generator().manual_seed(cfg.seed)

    def rnd(*shape, std=0.02):
        return (torch.randn(*shape, generator=g) * std).to(dtype).to(device)

    def proj(n_in, n_out):   # stored [in, out], so x @ w needs no transposed operand
        return rnd(n_in, n_out)

    def ones(n):
        return torch.ones(n, dtype=dtype, device=device)

    layers = []
    for _ in range(cfg.layers):
        layers.append(dict(
            ln_in=ones(cfg.hidden), ln_post=ones(cfg.hidden),
            wq=proj(cfg.hidden, cfg.heads * cfg.head_dim), wk=proj(cfg.hidden, cfg.kv_heads * cfg.head_dim),
            wv=proj(cfg.hidden, cfg.kv_heads * cfg.head_dim), wo=proj(cfg.heads * cfg.head_dim, cfg.hidden),
            q_norm=ones(cfg.head_dim), k_norm=ones(cfg.head_dim),
            wg=proj(cfg.hidden, cfg.intermediate), wu=proj(cfg.hidden, cfg.intermediate),
            wd=proj(cfg.intermediate, cfg.hidden)))
    return dict(embed=rnd(cfg.vocab, cfg.hidden), ln_final=ones(cfg.hidden), layers=layers,
                lm_head=(torch.randn(cfg.hidden, cfg.vocab, generator=g) * cfg.lm_head_std).to(device))


def rms_norm(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)).to(x.dtype) * w


def rope(x, positions, theta):
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, device=x.device, dtype=torch.float32) / d))
    ang = positions.float()[:, None] * inv[None, :]
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
    x1, x2 = x.float()[..., : d // 2], x.float()[..., d // 2:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


@dataclass
class StepContext:
    is_prefill: bool
    slot_mapping: torch.Tensor          # int32 [T]
    block_tables: torch.Tensor          # int32 [B, max_blocks]
    cu_seqlens_q: torch.Tensor = None   # int32 [B + 1]
    cu_seqlens_k: torch.Tensor = None
    max_q: int = 0
    max_k: int = 0
    context_lens: torch.Tensor = None   # int32 [B] (decode)
    q_lens: list = field(default_factory=list)
    k_lens: list = field(default_factory=list)


def native_attention(q, k, v, k_cache, v_cache, ctx, scale):
    fa.store_kvcache(k, v, k_cache, v_cache, ctx.slot_mapping)
    if ctx.is_prefill:
        return fa.flash_attn_varlen_func(q, k_cache, v_cache, ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.max_q,
                                         ctx.max_k, softmax_scale=scale, causal=True, block_table=ctx.block_tables)
    return fa.flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache, cache_seqlens=ctx.context_lens,
                                      block_table=ctx.block_tables, softmax_scale=scale, causal=True).squeeze(1)


def sdpa_attention(q, k, v, k_cache, v_cache, ctx, scale):
    """Timing baseline: index_copy_ slot writes and per-request torch SDPA (flash / memory-efficient
    backends, fp16, lower-right causal bias, GQA) over the gathered pages."""
    from compare_sdpa import sdpa_gqa
    slots = ctx.slot_mapping.long()
    k_cache.flatten(0, 1).index_copy_(0, slots, k)
    v_cache.flatten(0, 1).index_copy_(0, slots, v)
    outs, start = [], 0
    tables = ctx.block_tables.long()
    for b, (ql, kl) in enumerate(zip(ctx.q_lens, ctx.k_lens)):
        blocks = tables[b, : math.ceil(kl / PAGE)]
        key = k_cache[blocks].flatten(0, 1)[:kl].transpose(0, 1).unsqueeze(0).contiguous()
        val = v_cache[blocks].flatten(0, 1)[:kl].transpose(0, 1).unsqueeze(0).contiguous()
        query = q[start:start + ql].transpose(0, 1).unsqueeze(0).contiguous()
        outs.append(sdpa_gqa(query, key, val, ql, kl).squeeze(0).transpose(0, 1))
        start += ql
    return torch.cat(outs)


def reference_attention(q, k, v, k_cache, v_cache, ctx, scale):
    """index_copy_ slot writes, per-request page gather, fp32 softmax(QK^T)V, lower-right causal."""
    slots = ctx.slot_mapping.long()
    k_cache.flatten(0, 1).index_copy_(0, slots, k)
    v_cache.flatten(0, 1).index_copy_(0, slots, v)
    outs, start = [], 0
    group = q.shape[1] // k.shape[1]
    tables = ctx.block_tables.long()
    for b, (ql, kl) in enumerate(zip(ctx.q_lens, ctx.k_lens)):
        blocks = tables[b, : math.ceil(kl / PAGE)]
        key = k_cache[blocks].flatten(0, 1)[:kl].float().repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
        val = v_cache[blocks].flatten(0, 1)[:kl].float().repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
        query = q[start:start + ql].float().transpose(0, 1).contiguous()
        scores = torch.matmul(query, key.transpose(1, 2).contiguous()) * scale        # [H, ql, kl]
        row = torch.arange(ql, device=q.device)[:, None] + (kl - ql)
        scores = scores.masked_fill(torch.arange(kl, device=q.device)[None, :] > row, float("-inf"))
        out = torch.matmul(torch.softmax(scores, dim=-1), val)                          # [H, ql, D]
        outs.append(out.transpose(0, 1).to(q.dtype))
        start += ql
    return torch.cat(outs)


class Model:
    def __init__(self, cfg, weights, attention, num_blocks, device):
        self.cfg, self.w, self.attention = cfg, weights, attention
        shape = (num_blocks, PAGE, cfg.kv_heads, cfg.head_dim)
        self.caches = [(torch.zeros(shape, dtype=torch.float16, device=device),
                        torch.zeros(shape, dtype=torch.float16, device=device)) for _ in range(cfg.layers)]
        self.scale = cfg.head_dim ** -0.5

    def forward(self, ids, positions, ctx, last_index):
        cfg, T = self.cfg, ids.shape[0]
        x = self.w["embed"][ids]
        for lw, (kc, vc) in zip(self.w["layers"], self.caches):
            h = rms_norm(x, lw["ln_in"], cfg.eps)
            q = (h @ lw["wq"]).view(T, cfg.heads, cfg.head_dim)
            k = (h @ lw["wk"]).view(T, cfg.kv_heads, cfg.head_dim)
            v = (h @ lw["wv"]).view(T, cfg.kv_heads, cfg.head_dim).contiguous()
            q = rope(rms_norm(q, lw["q_norm"], cfg.eps), positions, cfg.rope_theta).contiguous()
            k = rope(rms_norm(k, lw["k_norm"], cfg.eps), positions, cfg.rope_theta).contiguous()
            o = self.attention(q, k, v, kc, vc, ctx, self.scale)
            x = x + o.reshape(T, -1) @ lw["wo"]
            h = rms_norm(x, lw["ln_post"], cfg.eps)
            x = x + (torch.nn.functional.silu(h @ lw["wg"]) * (h @ lw["wu"])) @ lw["wd"]
        x = rms_norm(x[last_index], self.w["ln_final"], cfg.eps)
        return x.float() @ self.w["lm_head"]


class Sequence:
    def __init__(self, sid, prompt, max_tokens):
        self.sid, self.tokens, self.prompt_len, self.max_tokens = sid, list(prompt), len(prompt), max_tokens
        self.blocks = []            # physical block ids
        self.computed = 0           # tokens whose K/V are in the cache
        self.cached = 0             # of which reused from the prefix cache

    @property
    def generated(self):
        return len(self.tokens) - self.prompt_len

    def done(self):
        return self.generated >= self.max_tokens


class BlockManager:
    """Free list plus hash chains over full blocks; a freed block keeps its hash until reused."""

    def __init__(self, num_blocks):
        self.free = list(range(num_blocks))
        self.ref = [0] * num_blocks
        self.hash_of = [None] * num_blocks
        self.by_hash = {}

    def _take(self):
        blk = self.free.pop(0)
        if self.hash_of[blk] is not None:
            self.by_hash.pop(self.hash_of[blk], None)
            self.hash_of[blk] = None
        self.ref[blk] = 1
        return blk

    def can_allocate(self, n):
        return len(self.free) >= n

    def allocate(self, seq):
        """Blocks for the whole current sequence; full blocks found in the cache are reused.  At least
        one token is always recomputed so the step yields logits."""
        n = math.ceil(len(seq.tokens) / PAGE)
        usable = (len(seq.tokens) - 1) // PAGE
        h, hits = None, 0
        for i in range(n):
            chunk = tuple(seq.tokens[i * PAGE:(i + 1) * PAGE])
            h = hash((h, chunk)) if len(chunk) == PAGE else None
            blk = self.by_hash.get(h) if (h is not None and i < usable and hits == i) else None
            if blk is not None:
                if self.ref[blk] == 0:
                    self.free.remove(blk)
                self.ref[blk] += 1
                hits += 1
            else:
                blk = self._take()
                if h is not None:
                    self.hash_of[blk] = h
                    self.by_hash[h] = blk
            seq.blocks.append(blk)
        seq.computed = seq.cached = hits * PAGE
        return hits

    def release(self, seq):
        for blk in reversed(seq.blocks):
            self.ref[blk] -= 1
            if self.ref[blk] == 0:
                self.free.append(blk)
        seq.blocks, seq.computed, seq.cached = [], 0, 0

    def append_slot(self, seq):
        """Room for one more token; False when a new block is needed and none is free."""
        if len(seq.tokens) > len(seq.blocks) * PAGE:
            if not self.free:
                return False
            seq.blocks.append(self._take())
        return True


class DecodeGraphs:
    """Decode steps captured once per batch size (HIP graphs through torch.cuda.CUDAGraph) and
    replayed with the step's inputs copied into static buffers.  Rows past the real batch are padding:
    slot -1 (no cache write), length 1, outputs ignored.  The attention calls read no device values
    on the host, which is what makes the step capturable."""

    def __init__(self, model, max_bs, num_blocks, device):
        self.model = model
        self.sizes = [b for b in (1, 2, 4, 8, 16, 32) if b < max_bs] + [max_bs]
        self.ids = torch.zeros(max_bs, dtype=torch.int64, device=device)
        self.pos = torch.zeros(max_bs, dtype=torch.int64, device=device)
        self.slots = torch.full((max_bs,), -1, dtype=torch.int32, device=device)
        self.tables = torch.zeros(max_bs, num_blocks, dtype=torch.int32, device=device)
        self.lens = torch.ones(max_bs, dtype=torch.int32, device=device)
        self.rows = torch.arange(max_bs, device=device)
        self.graphs, self.out = {}, {}

    def _forward(self, bs):
        ctx = StepContext(False, self.slots[:bs], self.tables[:bs], context_lens=self.lens[:bs], max_q=1,
                          max_k=self.tables.shape[1] * PAGE)
        return self.model.forward(self.ids[:bs], self.pos[:bs], ctx, self.rows[:bs])

    def _capture(self, bs):
        main = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            for _ in range(2):
                self._forward(bs)
        main.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.out[bs] = self._forward(bs)
        self.graphs[bs] = graph

    def run(self, ids, pos, slots, tables, lens):
        n = ids.shape[0]
        bs = next(b for b in self.sizes if b >= n)
        if bs not in self.graphs:
            self.slots.fill_(-1)
            self.lens.fill_(1)
            self._capture(bs)
        self.ids[:n] = ids
        self.pos[:n] = pos
        self.slots[:n] = slots
        self.slots[n:bs] = -1
        self.tables[:n] = 0
        self.tables[:n, : tables.shape[1]] = tables
        self.lens[:n] = lens
        self.lens[n:bs] = 1
        self.graphs[bs].replay()
        return self.out[bs][:n]


class Engine:
    def __init__(self, model, num_blocks, max_num_seqs, max_num_batched_tokens, device, graphs=False):
        self.model, self.device = model, device
        self.graphs = DecodeGraphs(model, max_num_seqs, num_blocks, device) if graphs else None
        self.bm = BlockManager(num_blocks)
        self.max_num_seqs, self.budget = max_num_seqs, max_num_batched_tokens
        self.waiting, self.running = [], []
        self.counters = {"prefix_hits": 0, "preemptions": 0, "sample_calls": 0, "prefill_steps": 0, "decode_steps": 0}

    def add(self, seq):
        self.waiting.append(seq)

    def _tables(self, seqs):
        width = max(len(s.blocks) for s in seqs)
        t = torch.zeros(len(seqs), width, dtype=torch.int32)
        for i, s in enumerate(seqs):
            t[i, : len(s.blocks)] = torch.tensor(s.blocks, dtype=torch.int32)
        return t

    def _slots(self, seq, lo, hi):
        pos = torch.arange(lo, hi)
        blocks = torch.tensor(seq.blocks, dtype=torch.int64)
        return blocks[pos // PAGE] * PAGE + pos % PAGE

    def _schedule_prefill(self):
        batch, used = [], 0
        while self.waiting and len(self.running) + len(batch) < self.max_num_seqs and used < self.budget:
            seq = self.waiting[0]
            if not seq.blocks:
                if not self.bm.can_allocate(math.ceil(len(seq.tokens) / PAGE)):
                    break
                hits = self.bm.allocate(seq)
                self.counters["prefix_hits"] += int(hits > 0)
            take = min(len(seq.tokens) - seq.computed, self.budget - used)
            batch.append((seq, seq.computed, seq.computed + take))
            used += take
            if seq.computed + take < len(seq.tokens):
                break                                   # the chunk budget is spent on this prompt
            self.waiting.pop(0)
        return batch

    def step(self, sampler):
        dev = self.device
        batch = self._schedule_prefill()
        if batch:
            self.counters["prefill_steps"] += 1
            seqs = [s for s, _, _ in batch]
            q_lens = [hi - lo for _, lo, hi in batch]
            k_lens = [hi for _, _, hi in batch]
            ids = torch.cat([torch.tensor(s.tokens[lo:hi]) for s, lo, hi in batch]).to(dev)
            pos = torch.cat([torch.arange(lo, hi) for _, lo, hi in batch]).to(dev)
            slots = torch.cat([self._slots(s, lo, hi) for s, lo, hi in batch]).to(dev, torch.int32)
            cuq = torch.tensor(list(itertools.accumulate(q_lens, initial=0)), dtype=torch.int32, device=dev)
            cuk = torch.tensor(list(itertools.accumulate(k_lens, initial=0)), dtype=torch.int32, device=dev)
            ctx = StepContext(True, slots, self._tables(seqs).to(dev), cuq, cuk, max(q_lens), max(k_lens),
                              q_lens=q_lens, k_lens=k_lens)
            logits = self.model.forward(ids, pos, ctx, cuq[1:].long() - 1)
            finished = []
            for i, (s, lo, hi) in enumerate(batch):
                s.computed = hi
                if hi == len(s.tokens):
                    finished.append(i)
                    self.running.append(s)
            if finished:
                choices = sampler(logits[finished], [batch[i][0] for i in finished])
                for i, tok in zip(finished, choices):
                    batch[i][0].tokens.append(int(tok))
            self._retire()
            return True
        if not self.running:
            return False
        # Decode: every running sequence gets one slot; when blocks run out the last running sequence
        # is preempted (its blocks freed, recomputed by a later prefill), possibly the one asking.
        seqs, i = [], 0
        while i < len(self.running):
            s = self.running[i]
            if self.bm.append_slot(s):
                seqs.append(s)
                i += 1
                continue
            victim = self.running.pop()       # index >= i, so never one already in seqs
            self.bm.release(victim)
            self.waiting.insert(0, victim)
            self.counters["preemptions"] += 1
        if not seqs:
            return True
        self.counters["decode_steps"] += 1
        ids = torch.tensor([s.tokens[-1] for s in seqs], device=dev)
        pos = torch.tensor([len(s.tokens) - 1 for s in seqs], device=dev)
        slots = torch.cat([self._slots(s, len(s.tokens) - 1, len(s.tokens)) for s in seqs]).to(dev, torch.int32)
        lens = [len(s.tokens) for s in seqs]
        tables = self._tables(seqs).to(dev)
        lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
        if self.graphs is not None:
            logits = self.graphs.run(ids, pos, slots, tables, lens_t)
        else:
            ctx = StepContext(False, slots, tables, context_lens=lens_t, q_lens=[1] * len(seqs), k_lens=lens,
                              max_q=1, max_k=max(lens))
            logits = self.model.forward(ids, pos, ctx, torch.arange(len(seqs), device=dev))
        for s in seqs:
            s.computed = len(s.tokens)
        for s, tok in zip(seqs, sampler(logits, seqs)):
            s.tokens.append(int(tok))
        self._retire()
        return True

    def _retire(self):
        for s in [s for s in self.running if s.done()]:
            self.running.remove(s)
            self.bm.release(s)

    def generate(self, prompts, max_tokens, sampler, first_sid=0):
        seqs = [Sequence(first_sid + i, p, max_tokens) for i, p in enumerate(prompts)]
        for s in seqs:
            self.add(s)
        while self.step(sampler):
            pass
        return [s.tokens[s.prompt_len:] for s in seqs]


def kl_rows(ref, act):
    ref_logp = ref.double().log_softmax(-1)
    act_logp = act.double().log_softmax(-1)
    return (ref_logp.exp() * (ref_logp - act_logp)).sum(-1)


def run_case(cfg, weights, settings, batches, backend, device, expected=None, graphs=False):
    """One engine run; with `expected` the sampler is teacher-forced and logits are compared."""
    model = Model(cfg, weights, backend, settings["num_blocks"], device)
    eng = Engine(model, settings["num_blocks"], settings["max_num_seqs"], settings["max_num_batched_tokens"], device,
                 graphs=graphs)
    trace, errors = [], []

    def sampler(logits, seqs):
        if not torch.isfinite(logits).all():
            raise AssertionError("non-finite logits")
        choices = logits.argmax(-1).cpu()
        index = eng.counters["sample_calls"]
        eng.counters["sample_calls"] += 1
        if expected is None:
            trace.append((logits.cpu(), choices))
            return choices.tolist()
        ref, tokens = expected[index]
        act = logits.cpu()
        kl = kl_rows(ref, act)
        # A differing greedy choice counts only where the reference's top-2 gap exceeds twice that row's
        # largest logit difference (closer ties are not decided by either implementation's rounding).
        top2 = ref.topk(2, dim=-1).values
        decided = (top2[:, 0] - top2[:, 1]) > 2 * (act - ref).abs().max(dim=-1).values
        differ = choices != tokens
        errors.append({"kl_max": float(kl.max().clamp_min(0)), "max_abs": float((act - ref).abs().max()),
                       "greedy_matches": bool(not differ.any()),
                       "greedy_mismatches_decided": int((differ & decided).sum())})
        return tokens.tolist()

    outputs, sid = [], 0
    t0 = time.perf_counter()
    for prompts, max_tokens in batches:
        outputs.append(eng.generate(prompts, max_tokens, sampler, first_sid=sid))
        sid += len(prompts)
    torch.cuda.synchronize()
    return {"counters": dict(eng.counters), "outputs": outputs, "errors": errors,
            "elapsed_s": time.perf_counter() - t0}, trace


def cases():
    pattern = [(7 * i + 3) % 997 + 11 for i in range(41)]

    def tokens(n, offset=0):
        return [pattern[(i + offset) % len(pattern)] for i in range(n)]

    base = dict(max_num_seqs=4, max_num_batched_tokens=1024, num_blocks=16)
    return [
        ("normal", base, [([tokens(5), tokens(9, 5)], 16)]),
        ("cross-page", base, [([tokens(255)], 16)]),
        ("shared-prefix", base, [([tokens(520)], 8), ([tokens(512) + tokens(9, 2), tokens(512) + tokens(13, 4)], 16)]),
        ("chunked-prefill", {**base, "max_num_batched_tokens": 128}, [([tokens(777)], 16)]),
        ("preemption", {**base, "num_blocks": 2, "max_num_batched_tokens": 512}, [([tokens(255), tokens(255, 3)], 16)]),
    ]


def check(name, ref, native, batches):
    """The acceptance criteria of one case; returns a list of failures."""
    bad = []
    for i, e in enumerate(native["errors"]):
        if not (e["kl_max"] <= KL_LIMIT):
            bad.append(f"{name}: KL {e['kl_max']:.2e} at sampler call {i}")
        if e["greedy_mismatches_decided"]:
            bad.append(f"{name}: greedy choice differs at sampler call {i}")
    if ref["outputs"] != native["outputs"]:
        bad.append(f"{name}: outputs differ")
    c = native["counters"]
    if name == "shared-prefix" and c["prefix_hits"] < 2:
        bad.append(f"{name}: expected prefix-cache hits, got {c}")
    if name == "preemption" and c["preemptions"] < 1:
        bad.append(f"{name}: expected a preemption, got {c}")
    expected_tokens = sum(len(prompts) * max_tokens for prompts, max_tokens in batches)
    if len(native["errors"]) == 0 or sum(len(o) for outs in native["outputs"] for o in outs) != expected_tokens:
        bad.append(f"{name}: not every request produced its tokens ({native['outputs']})")
    if name == "chunked-prefill" and c["prefill_steps"] < 7:
        bad.append(f"{name}: expected chunked prefill steps, got {c}")
    return bad


def run_all(cfg, device, only=None):
    weights = init_weights(cfg, device)
    report = {"model": cfg.__dict__, "kl_limit": KL_LIMIT, "page": PAGE, "cases": []}
    failures = []
    with torch.inference_mode():
        for name, settings, batches in cases():
            if only and name != only:
                continue
            ref, trace = run_case(cfg, weights, settings, batches, reference_attention, device)
            native, _ = run_case(cfg, weights, settings, batches, native_attention, device, expected=trace)
            graphed, _ = run_case(cfg, weights, settings, batches, native_attention, device, expected=trace,
                                  graphs=True)
            bad = check(name, ref, native, batches) + [f"{b} (graph-captured decode)" for b in
                                                       check(name, ref, graphed, batches)]
            failures += bad
            report["cases"].append({
                "name": name, "settings": settings, "counters": native["counters"],
                "sampler_calls": len(native["errors"]),
                "kl_max": max((e["kl_max"] for e in native["errors"]), default=0.0),
                "logit_max_abs": max((e["max_abs"] for e in native["errors"]), default=0.0),
                "greedy_matches": all(e["greedy_matches"] for e in native["errors"]),
                "greedy_mismatches_decided": sum(e["greedy_mismatches_decided"] for e in native["errors"]),
                "graph_kl_max": max((e["kl_max"] for e in graphed["errors"]), default=0.0),
                "reference_s": ref["elapsed_s"], "native_s": native["elapsed_s"], "passed": not bad})
            print(name, json.dumps(report["cases"][-1]["counters"]), "kl_max",
                  f"{report['cases'][-1]['kl_max']:.2e}", "PASS" if not bad else "FAIL", flush=True)
    report["passed"] = not failures
    return report, failures


def performance(cfg, device, prompt_len=1024, generated=128, rounds=3):
    """Greedy generation throughput of the engine with native vs SDPA attention, batch 1 and 4
    (the shape of the reference's benchmarks/bench_nanovllm_optimization.py:202-260: 1024-token
    prompts, 128 new tokens, a warmup generation on prompts that share no cached prefix)."""
    weights = init_weights(cfg, device)
    settings = dict(max_num_seqs=4, max_num_batched_tokens=4096, num_blocks=32)
    pattern = [(7 * i + 3) % 997 + 11 for i in range(41)]
    rows = []

    def sampler(logits, seqs):
        return logits.argmax(-1).tolist()

    for batch in (1, 4):
        prompts = [[pattern[(i + off) % len(pattern)] for i in range(prompt_len)] for off in range(batch)]
        warm = [[1000 + j] + p[1:] for j, p in enumerate(prompts)]
        row = {"batch": batch, "prompt_tokens": prompt_len, "generated_tokens": generated}
        for label, backend, graphs in (("sdpa", sdpa_attention, False), ("native", native_attention, False),
                                       ("native_graph", native_attention, True)):
            rates = []
            for _ in range(rounds):
                model = Model(cfg, weights, backend, settings["num_blocks"], device)
                eng = Engine(model, settings["num_blocks"], settings["max_num_seqs"],
                             settings["max_num_batched_tokens"], device, graphs=graphs)
                eng.generate(warm, 16, sampler)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                outs = eng.generate(prompts, generated, sampler, first_sid=100)
                torch.cuda.synchronize()
                rates.append(sum(len(o) for o in outs) / (time.perf_counter() - t0))
                del model, eng
            row[label + "_tokens_per_s"] = sorted(rates)[len(rates) // 2]
        row["speedup"] = row["native_tokens_per_s"] / row["sdpa_tokens_per_s"]
        row["graph_speedup"] = row["native_graph_tokens_per_s"] / row["sdpa_tokens_per_s"]
        print("performance", json.dumps(row), flush=True)
        rows.append(row)
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--case")
    ap.add_argument("--performance", action="store_true", help="also time generation, native vs SDPA")
    opts = ap.parse_args()
    if not torch.cuda.is_available():
        sys.exit("validate_engine.py needs a GPU")
    cfg = ModelConfig(layers=opts.layers)
    report, failures = run_all(cfg, torch.device("cuda", 0), opts.case)
    if opts.performance:
        with torch.inference_mode():
            report["performance"] = performance(cfg, torch.device("cuda", 0))
    report["device"] = torch.cuda.get_device_name(0)
    report["torch"] = torch.__version__
    opts.output.parent.mkdir(parents=True, exist_ok=True)
    opts.output.write_text(json.dumps(report, indent=2) + "\n")
    if failures:
        sys.exit("\n".join(failures))


if __name__ == "__main__":
    main()
