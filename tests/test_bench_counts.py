"""bench.py's algorithmic work counts, checked on the CPU: the closed-form
count of visible (query, key) pairs under lower-right causality against the
oracle's per-row count (oracle/attention.py flops(), itself pinned to a
brute-force enumeration in test_oracle_attention.py)."""
import random

import bench
from oracle.attention import flops


def test_causal_pairs_match_the_oracle_count():
    rng = random.Random(7)
    cases = [([1], [1]), ([0, 3], [5, 0]), ([7, 100], [7, 100]), ([300], [40]), ([40], [300])]
    for _ in range(500):
        n = rng.randint(1, 6)
        cases.append(([rng.randint(0, 400) for _ in range(n)], [rng.randint(0, 400) for _ in range(n)]))
    for q_lens, k_lens in cases:
        assert bench.causal_pairs(q_lens, k_lens) * 2 * 2 == flops(q_lens, k_lens, 1, 1, 1), (q_lens, k_lens)


def test_config2_pair_count_is_the_bench_flop_basis():
    lengths = [256, 4096, 1000]
    assert bench.causal_pairs(lengths, lengths) == sum(n * (n + 1) // 2 for n in lengths)
