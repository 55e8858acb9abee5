"""ctypes binding of libfa_gfx950.so (declared in include/fa_gfx950.h).

The structures below mirror the C structs field for field; `load()` checks
their sizes against `fa_struct_sizes()` so a layout mismatch fails at import
of the first kernel call instead of corrupting arguments.  There is no CPU or
pure-PyTorch fallback: if the library is missing or a call fails, a
RuntimeError is raised.
"""
import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libfa_gfx950.so"

F16, BF16, F32, E4M3 = 0, 1, 2, 3
I32, I64 = 0, 1

DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32,
              torch.float8_e4m3fn: E4M3}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


def _arr(t, n):
    return t * n


class StoreDesc(ctypes.Structure):
    _fields_ = [("x", _p), ("cache", _p), ("scale", _p),
                ("x_dtype", _i32), ("cache_dtype", _i32),
                ("heads", _i64), ("dim", _i64),
                ("x_stride", _arr(_i64, 3)), ("cache_stride", _arr(_i64, 4)),
                ("scale_stride", _i64)]


class StoreArgs(ctypes.Structure):
    _fields_ = [("kv", _arr(StoreDesc, 2)), ("slots", _p), ("slot_dtype", _i32), ("_pad0", _i32),
                ("slot_stride", _i64), ("tokens", _i64), ("page_size", _i64), ("num_pages", _i64)]


class AppendArgs(ctypes.Structure):
    _fields_ = [("kv", _arr(StoreDesc, 2)), ("x_batch_stride", _arr(_i64, 2)),
                ("lengths", _p), ("batch_index", _p), ("block_table", _p),
                ("batch", _i64), ("new_tokens", _i64), ("page_size", _i64),
                ("num_blocks", _i64), ("table_rows", _i64), ("table_cols", _i64)]


class RotaryArgs(ctypes.Structure):
    _fields_ = [("x", _p), ("out", _p), ("cos_table", _p), ("sin_table", _p), ("lengths", _p),
                ("dtype", _i32), ("interleaved", _i32), ("advance", _i32), ("_pad0", _i32),
                ("batch", _i64), ("seq", _i64), ("heads", _i64), ("dim", _i64),
                ("half_rot", _i64), ("table_rows", _i64), ("x_stride", _arr(_i64, 4))]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", _p), ("k", _p), ("v", _p), ("out", _p), ("lse", _p),
                ("q_dtype", _i32), ("k_dtype", _i32), ("v_dtype", _i32), ("out_dtype", _i32),
                ("total_q", _i64), ("heads_q", _i64), ("heads_k", _i64),
                ("head_dim_qk", _i64), ("head_dim_v", _i64), ("batch", _i64),
                ("page_size", _i64), ("max_seqlen_q", _i64), ("max_seqlen_k", _i64),
                ("q_stride", _arr(_i64, 3)), ("k_stride", _arr(_i64, 4)), ("v_stride", _arr(_i64, 4)),
                ("out_stride", _arr(_i64, 3)), ("lse_stride", _arr(_i64, 2)),
                ("cu_seqlens_q", _p), ("cu_q_stride", _i64),
                ("cu_seqlens_k", _p), ("cu_k_stride", _i64),
                ("seqused_k", _p), ("used_k_stride", _i64),
                ("block_table", _p), ("bt_stride", _arr(_i64, 2)),
                ("leftpad_k", _p), ("leftpad_stride", _i64),
                ("causal", _i32), ("window_left", _i32), ("window_right", _i32),
                ("mask_kind", _i32), ("mask_window", _i32), ("mask_clamp", _i32),
                ("causal_by_batch", _p), ("causal_stride", _i64),
                ("mask_ranges", _p), ("ranges_stride", _arr(_i64, 2)),
                ("mask_prefix", _p), ("prefix_stride", _i64),
                ("mask_window_len", _p),
                ("softmax_scale", _f32), ("softcap", _f32),
                ("alibi", _p), ("alibi_stride", _arr(_i64, 2)),
                ("sinks", _p), ("sink_stride", _i64),
                ("q_descale", _p), ("q_descale_stride", _arr(_i64, 2)),
                ("k_descale", _p), ("k_descale_stride", _arr(_i64, 2)),
                ("v_descale", _p), ("v_descale_stride", _arr(_i64, 2)),
                ("num_splits", _i32), ("split_span", _i32),
                ("partial_out", _p), ("partial_lse", _p),
                ("flags", _i32), ("_pad1", _i32)]


class MergePairArgs(ctypes.Structure):
    _fields_ = [("out", _p), ("a", _p), ("b", _p), ("a_lse", _p), ("b_lse", _p), ("out_lse", _p),
                ("dtype", _i32), ("_pad0", _i32),
                ("tokens", _i64), ("heads", _i64), ("dim", _i64),
                ("out_stride", _arr(_i64, 3)), ("a_stride", _arr(_i64, 3)), ("b_stride", _arr(_i64, 3)),
                ("a_lse_stride", _arr(_i64, 2)), ("b_lse_stride", _arr(_i64, 2)),
                ("out_lse_stride", _arr(_i64, 2))]


class MergePartialsArgs(ctypes.Structure):
    _fields_ = [("partial", _p), ("partial_lse", _p), ("out", _p), ("lse", _p),
                ("partial_dtype", _i32), ("out_dtype", _i32),
                ("splits", _i64), ("tokens", _i64), ("heads", _i64), ("dim", _i64),
                ("partial_stride", _arr(_i64, 4)), ("partial_lse_stride", _arr(_i64, 3)),
                ("out_stride", _arr(_i64, 3)), ("lse_stride", _arr(_i64, 2))]


STRUCTS = (StoreArgs, AppendArgs, RotaryArgs, AttnArgs, MergePairArgs, MergePartialsArgs)

# Entry points declared in include/fa_gfx950.h: name -> (argument struct or None, restype).
ENTRY_POINTS = {
    "fa_abi_version": (None, ctypes.c_int),
    "fa_struct_sizes": (None, None),
    "fa_last_error": (None, ctypes.c_char_p),
    "fa_store_kvcache": (StoreArgs, ctypes.c_int),
    "fa_append_kvcache": (AppendArgs, ctypes.c_int),
    "fa_rotary": (RotaryArgs, ctypes.c_int),
    "fa_decode_supported": (AttnArgs, ctypes.c_int),
    "fa_decode_fwd": (AttnArgs, ctypes.c_int),
    "fa_decode_fwd_noalloc": (AttnArgs, ctypes.c_int),
    "fa_prefill_supported": (AttnArgs, ctypes.c_int),
    "fa_prefill_fwd": (AttnArgs, ctypes.c_int),
    "fa_attn_fwd": (AttnArgs, ctypes.c_int),
    "fa_merge_pair": (MergePairArgs, ctypes.c_int),
    "fa_merge_partials": (MergePartialsArgs, ctypes.c_int),
}

ABI_VERSION = 3
FLAG_SKIP_SINGLE_QUERY = 1
DECODE_SCRATCH_BYTES = 32 << 20   # FA_DECODE_SCRATCH_BYTES
_lib = None


def load():
    """Load libfa_gfx950.so once (torch is imported first so the library binds to
    torch's HIP runtime, which shares the libamdhip64.so.7 soname)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH.name} is not built; run __graft_entry__.build() "
                           "(make -C flash-attn-mps_amd/csrc)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (struct, restype) in ENTRY_POINTS.items():
        fn = getattr(lib, name)
        fn.restype = restype
        if name == "fa_struct_sizes":
            fn.argtypes = [ctypes.POINTER(_i64)]
        elif struct is not None:
            fn.argtypes = ([ctypes.POINTER(struct)] if name.endswith("supported")
                           else [ctypes.POINTER(struct), _p])
        else:
            fn.argtypes = []
    if lib.fa_abi_version() != ABI_VERSION:
        raise RuntimeError("libfa_gfx950.so ABI version mismatch")
    sizes = (_i64 * 6)()
    lib.fa_struct_sizes(sizes)
    for struct, size in zip(STRUCTS, sizes):
        if ctypes.sizeof(struct) != size:
            raise RuntimeError(f"{struct.__name__}: ctypes size {ctypes.sizeof(struct)} != C size {size}")
    _lib = lib
    return lib


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def call(name, args, device):
    lib = load()
    rc = getattr(lib, name)(ctypes.byref(args), stream_of(device))
    if rc != 0:
        raise RuntimeError(f"{name} failed ({rc}): {lib.fa_last_error().decode()}")


def supported(name, args):
    return bool(getattr(load(), name)(ctypes.byref(args)))


def ptr(t):
    return None if t is None else t.data_ptr()


def strides(t, n):
    s = list(t.stride())
    return (s + [0] * n)[:n]
