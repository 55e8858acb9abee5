"""CPU oracle for flash_attn_mps_amd -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of SuperMarioYL/flash-attn-mps
for the attention / cache / merge hot path.  It is the checker that the HIP
kernels are compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product package
never does, and has no CPU fallback.

Modules and what pins each one (tests/test_oracle_*.py, all CPU-only):
  attention.py  -- tests/reference.py:6-90 restated.  Pinned by
                   tests/oracle_pins.py: torch SDPA for varlen/GQA/causal/
                   windows/ALiBi/default scale, closed forms (zero query,
                   single key, two-key softcap), identities (sinks,
                   descales, paged = packed, leftpad, causal_by_batch, mask
                   kinds at extreme parameters), the empty-KV golden values of
                   test_attention_core.py:52-63 and tests/golden/sdpa.npz.
                   tests/test_oracle_mutants.py plants 20 mistakes and shows
                   each is caught.  flops() is checked by brute force.
  merge.py      -- kernels/merge.metal:9-58 restated; pinned by log-add-exp
                   closed forms, the extreme-LSE table of test_merge.py:14-27
                   (tests/golden/merge.npz) and the NaN-payload rules.
  cache.py      -- kernels/cache.metal:20-76 restated; pinned against
                   index_copy_ scatter, torch's float8_e4m3fn cast, literal
                   landing positions of test_cache.py:57-75 and complex-number
                   rotation.
  fp8.py        -- ctypes binding of fp8_e4m3.c (kernels/cache.metal:8-18,
                   attention.metal:4-10); pinned against torch's cast for all
                   256 decode codes and ~1M float32 encode inputs, and the
                   RNE/saturation table of test_cache.py:39-54
                   (tests/golden/e4m3.npz).
No oracle function is left "parity unpinned".
"""
