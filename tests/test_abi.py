"""C-ABI checks that need no GPU: libfa_gfx950.so loads, exports exactly the
entry points declared in include/fa_gfx950.h, its argument structs have the
sizes the ctypes mirrors assume, and invalid arguments are rejected before
any HIP call."""
import ctypes
import re
from pathlib import Path

import pytest

from flash_attn_mps_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "fa_gfx950.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|void|const char\*)\s+(fa_\w+)\s*\(", text, re.M)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert names == sorted(_lib.ENTRY_POINTS), names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_struct_sizes_match_c_layout():
    lib = _lib.load()
    sizes = (ctypes.c_int64 * 6)()
    lib.fa_struct_sizes(sizes)
    assert [ctypes.sizeof(s) for s in _lib.STRUCTS] == list(sizes)
    assert lib.fa_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("name,struct", [
    ("fa_store_kvcache", _lib.StoreArgs), ("fa_append_kvcache", _lib.AppendArgs),
    ("fa_rotary", _lib.RotaryArgs), ("fa_attn_fwd", _lib.AttnArgs),
    ("fa_decode_fwd", _lib.AttnArgs), ("fa_prefill_fwd", _lib.AttnArgs),
    ("fa_merge_pair", _lib.MergePairArgs), ("fa_merge_partials", _lib.MergePartialsArgs),
])
def test_null_arguments_are_rejected_before_launch(name, struct):
    lib = _lib.load()
    args = struct()   # all pointers NULL
    if hasattr(args, "splits"):
        args.splits = 1
    rc = getattr(lib, name)(ctypes.byref(args), None)
    assert rc == 1, rc          # FA_ERR_INVALID
    assert lib.fa_last_error().decode().startswith(name)


def test_noalloc_decode_rejects_bad_arguments_before_any_hip_call():
    lib = _lib.load()
    assert lib.fa_decode_fwd_noalloc(None, None) == 1
    a = _lib.AttnArgs()
    a.num_splits = 1                        # explicit plan: NULL tensors fail validation
    assert lib.fa_decode_fwd_noalloc(ctypes.byref(a), None) == 1
    assert lib.fa_last_error().decode().startswith("fa_decode_fwd_noalloc")
    a.partial_out = 4096                    # partials are library-owned
    assert lib.fa_decode_fwd_noalloc(ctypes.byref(a), None) == 1
    assert b"library-owned" in lib.fa_last_error()
    a.partial_out, a.num_splits = None, 0   # library plan: bad head counts, then an unsupported layout
    assert lib.fa_decode_fwd_noalloc(ctypes.byref(a), None) == 1
    assert b"head counts" in lib.fa_last_error()
    a.batch = a.heads_q = a.heads_k = 1
    assert lib.fa_decode_fwd_noalloc(ctypes.byref(a), None) == 2


def test_zero_kv_heads_are_refused_not_divided_by():
    """A supported-looking decode layout with heads_k = 0: the support query
    answers 0 and the no-allocation entry point returns FA_ERR_INVALID (the
    head-group arithmetic divides by heads_k)."""
    lib = _lib.load()
    a = _lib.AttnArgs()
    a.q_dtype = a.k_dtype = a.v_dtype = a.out_dtype = _lib.BF16
    a.head_dim_qk = a.head_dim_v = 128
    a.q_stride[2] = a.out_stride[2] = a.k_stride[3] = a.v_stride[3] = 1
    a.batch, a.heads_q, a.heads_k, a.max_seqlen_q = 1, 8, 0, 1
    assert not _lib.supported("fa_decode_supported", a)
    assert lib.fa_decode_fwd_noalloc(ctypes.byref(a), None) == 1


def test_supported_queries_reject_unsupported_combinations():
    a = _lib.AttnArgs()
    a.k_dtype = a.v_dtype = _lib.F32
    a.head_dim_qk = a.head_dim_v = 100
    a.heads_q = a.heads_k = 1
    assert not _lib.supported("fa_decode_supported", a)
    assert not _lib.supported("fa_prefill_supported", a)


def _paged_prefill_args(page_size, max_k):
    """A bf16 d128 paged-prefill layout (pointers only need 16-byte alignment here)."""
    a = _lib.AttnArgs()
    a.q_dtype = a.k_dtype = a.v_dtype = a.out_dtype = _lib.BF16
    a.head_dim_qk = a.head_dim_v = 128
    a.batch, a.heads_q, a.heads_k, a.total_q = 2, 8, 2, 128
    a.max_seqlen_q, a.max_seqlen_k = 64, max_k
    a.q = a.k = a.v = a.out = 1 << 20
    for name, strides in (("q_stride", (8 * 128, 128, 1)), ("out_stride", (8 * 128, 128, 1)),
                          ("k_stride", (page_size * 2 * 128, 2 * 128, 128, 1)),
                          ("v_stride", (page_size * 2 * 128, 2 * 128, 128, 1))):
        for i, s in enumerate(strides):
            getattr(a, name)[i] = s
    a.page_size, a.num_splits = page_size, 1
    a.window_left = a.window_right = -1
    return a


@pytest.mark.parametrize("page_size,max_k,ok", [(16, 4096, True), (256, 100000, True), (48, 96, False),
                                                (4160, 4160, True), (600, 512, True), (600, 601, False)])
def test_prefill_pages_are_powers_of_two_or_one_page_per_request(page_size, max_k, ok):
    """The MFMA prefill splits a position into page and slot with a shift:
    pages must be powers of two unless every key lies in the first page (a
    dense cache of any capacity seen through a one-column table)."""
    assert _lib.supported("fa_prefill_supported", _paged_prefill_args(page_size, max_k)) == ok
