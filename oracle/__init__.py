"""CPU oracle for flash_attn_mps_amd -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of SuperMarioYL/flash-attn-mps
for the attention / cache / merge hot path.  It is the checker that the HIP
kernels are compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product package
never does, and has no CPU fallback.

Modules and what pins each one (the pinning tests live in tests/test_oracle_*.py):
  attention.py  -- tests/reference.py:6-90 restated; pinned against
                   torch.nn.functional.scaled_dot_product_attention on the
                   feature-free subset, brute-force scalar loops for every mask,
                   window, softcap, ALiBi and sink rule, closed-form sink/LSE
                   identities and the empty-KV golden values.
  merge.py      -- kernels/merge.metal:9-58 restated; pinned by log-add-exp
                   closed forms and the extreme-LSE table of test_merge.py:14-27.
  cache.py      -- kernels/cache.metal:20-76 restated; pinned against
                   index_copy_ scatter, torch's float8_e4m3fn cast and the
                   rotary formula of test_cache.py:106-140.
  fp8.py        -- ctypes binding of fp8_e4m3.c (kernels/cache.metal:8-18,
                   attention.metal:4-10); pinned exhaustively against torch's
                   cast and the RNE/saturation table of test_cache.py:39-54.
"""
