"""FlashAttention inference for PyTorch-ROCm on AMD Instinct MI355X (gfx950).

A drop-in for the public API of flash_attn_mps (flash_attn_mps/__init__.py:3-29):
the FlashAttention-2 functions, ``store_kvcache`` and ``merge_attn_states``,
with the same names, signatures and tensor contracts, computed by hand-written
gfx950 HIP kernels in ``libfa_gfx950.so``.  The vLLM contract lives in
``flash_attn_mps_amd.vllm``.
"""

from .interface import (
    flash_attn_func,
    flash_attn_kvpacked_func,
    flash_attn_qkvpacked_func,
    flash_attn_varlen_func,
    flash_attn_varlen_kvpacked_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_with_kvcache,
)
from .vllm import merge_attn_states

__version__ = "0.2.0"


def store_kvcache(key, value, k_cache, v_cache, slot_mapping, *, k_scale=None, v_scale=None):
    """Write key/value [T, Hkv, D] rows to cache slots (slot // P, slot % P); slots < 0 are skipped."""
    from ._cache import store_kvcache as _store
    _store(key, value, k_cache, v_cache, slot_mapping, k_scale=k_scale, v_scale=v_scale)


__all__ = [
    "flash_attn_func", "flash_attn_kvpacked_func", "flash_attn_qkvpacked_func",
    "flash_attn_varlen_func", "flash_attn_varlen_kvpacked_func",
    "flash_attn_varlen_qkvpacked_func", "flash_attn_with_kvcache", "store_kvcache",
    "merge_attn_states",
]
