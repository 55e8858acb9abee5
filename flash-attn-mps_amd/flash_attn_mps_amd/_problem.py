"""One attention call in normal form, and the contract it must satisfy.

Every public entry point (dense, packed, varlen, KV-cache, vLLM) turns its
arguments into a :class:`Problem`: packed queries ``[T, Hq, Dqk]``, packed
``[Tk, Hkv, D]`` or paged ``[pages, P, Hkv, D]`` keys/values, int32 request
metadata, and the score/mask features.  :meth:`Problem.validate` then walks a
fixed table of contracts -- one :class:`Want` per tensor argument plus a few
scalar rules -- and raises on the first one broken, before anything is
enqueued on the GPU.

Error classes follow the drop-in contract of flash_attn_mps
(interface.py:37-147, _attention.py:95-126): ``ValueError`` for devices,
shapes, metadata and metadata dtypes; ``TypeError`` for unsupported element
types and mask objects; ``NotImplementedError`` for training features.
"""
from dataclasses import dataclass, field
from typing import Optional

import torch

ELEMENT_TYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float8_e4m3fn)
OUTPUT_TYPES = (torch.float16, torch.bfloat16, torch.float32)
MAX_HEAD_DIM = 512


@dataclass(frozen=True)
class MaskSpec:
    """A vLLM attention-mask semantic understood by the kernels (not a callback).

    kind 1: multimodal prefix (`mm_prefix_mask`), aux = ranges [T, 2], cu_seqlens_q [B+1];
    kind 2: rolling sliding window over a prefix (`rswa_mask`), aux = prefix [B], window [1].
    """

    kind: int
    sliding_window_left: int = -1
    clamp_prefix_to_window: bool = False


def reject_training(dropout_p=0.0, return_attn_probs=False, tensors=()):
    """The library is forward-only: no dropout, no probability output, no autograd."""
    if dropout_p:
        raise NotImplementedError(f"dropout_p={dropout_p}: only inference is implemented (dropout_p must be 0)")
    if return_attn_probs:
        raise NotImplementedError("return_attn_probs is not available; ask for return_softmax_lse=True instead")
    for t in tensors:
        if t is not None and t.requires_grad:
            raise NotImplementedError("tensors that require grad are not supported: there is no backward pass")


def on_gpu(t):
    return t.device.type == "cuda"


@dataclass(frozen=True)
class Want:
    """What a tensor argument must look like.

    shape: tuple of ints (``None`` = any extent), or a set of such tuples;
    dtypes: accepted element types (empty = any), with the error class raised
    for another type.
    """

    name: str
    shape: object = None
    dtypes: tuple = ()
    dtype_error: type = ValueError

    def _shape_ok(self, t):
        options = self.shape if isinstance(self.shape, (set, frozenset, list)) else [self.shape]
        for s in options:
            if s is None:
                return True
            if t.ndim == len(s) and all(e is None or e == n for e, n in zip(s, t.shape)):
                return True
        return False

    def check(self, t, device):
        if t is None:
            return
        if t.device != device:
            raise ValueError(f"{self.name} is on {t.device}; expected the queries' device {device}")
        if not self._shape_ok(t):
            raise ValueError(f"{self.name} has shape {tuple(t.shape)}; expected {self._describe()}")
        if self.dtypes and t.dtype not in self.dtypes:
            names = "/".join(str(d).replace("torch.", "") for d in self.dtypes)
            raise self.dtype_error(f"{self.name} is {str(t.dtype).replace('torch.', '')}; expected {names}")

    def _describe(self):
        options = self.shape if isinstance(self.shape, (set, frozenset, list)) else [self.shape]
        return " or ".join("[" + ", ".join("*" if e is None else str(e) for e in s) + "]" for s in options)


def _check(t, name, shape, dtypes, device, dtype_error=ValueError):
    """Want(name, shape, dtypes).check(t, device) for one exact shape, with
    the Want (and its message) built only when the tensor breaks it."""
    if t is None:
        return
    ts = t.shape
    if (t.device != device or len(ts) != len(shape) or any(e is not None and e != n for e, n in zip(shape, ts))
            or (dtypes and t.dtype not in dtypes)):
        Want(name, shape, dtypes, dtype_error).check(t, device)


@dataclass
class Problem:
    """Normalised arguments of one attention call (all tensors on one GPU).

    Lengths: request b owns query rows cu_q[b]:cu_q[b+1]; its keys are
    cu_k[b+1]-cu_k[b] rows from cu_k[b] (packed) or used_k[b] positions read
    through table[b] (paged, or a 1-column table of cache rows for a dense
    cache); leftpad[b] shifts where those positions sit in storage.
    """

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    cu_q: torch.Tensor
    max_q: int
    max_k: int
    cu_k: Optional[torch.Tensor] = None
    used_k: Optional[torch.Tensor] = None
    table: Optional[torch.Tensor] = None
    leftpad: Optional[torch.Tensor] = None
    scale: Optional[float] = None
    causal: object = False                  # bool, or a bool [B] tensor (vLLM dynamic causality)
    window: tuple = (-1, -1)
    softcap: float = 0.0
    alibi: Optional[torch.Tensor] = None
    sinks: Optional[torch.Tensor] = None
    q_descale: Optional[torch.Tensor] = None
    k_descale: Optional[torch.Tensor] = None
    v_descale: Optional[torch.Tensor] = None
    mask: Optional[MaskSpec] = None
    mask_aux: Optional[tuple] = None
    out: Optional[torch.Tensor] = None
    splits: int = 0
    deterministic: bool = False
    keep: list = field(default_factory=list)   # temporaries that must outlive the launch

    # ---- derived sizes
    @property
    def device(self):
        return self.q.device

    @property
    def batch(self):
        return self.cu_q.numel() - 1

    @property
    def tokens(self):
        return self.q.shape[0]

    @property
    def heads(self):
        return self.q.shape[1]

    @property
    def kv_heads(self):
        return self.k.shape[-2]

    @property
    def dim_qk(self):
        return self.q.shape[-1]

    @property
    def dim_v(self):
        return self.v.shape[-1]

    @property
    def paged(self):
        return self.k.ndim == 4

    @property
    def output_dtype(self):
        """FP8 queries produce fp16 (flash_attn_mps/_attention.py:120); others keep their type."""
        return torch.float16 if self.q.dtype == torch.float8_e4m3fn else self.q.dtype

    @property
    def visible_max(self):
        """Most keys a single query row can see (a left window clips max_k)."""
        left = self.window[0]
        return min(self.max_k, left + 1) if left >= 0 else self.max_k

    # ---- contract
    def validate(self):
        """Raise on the first broken contract (the checks run on every call,
        so each one is a plain test; messages are formatted only on failure)."""
        q, k, v = self.q, self.k, self.v
        reject_training(tensors=(q, k, v, self.alibi, self.sinks, self.q_descale, self.k_descale, self.v_descale,
                                 self.out))
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.device.type != "cuda":
                raise ValueError(f"{name} is on {t.device}; this library runs on a ROCm GPU ('cuda' device)")
        if q.ndim != 3:
            raise ValueError(f"q must be packed [tokens, heads, dim]; got {q.ndim} dims")
        if k.ndim not in (3, 4) or v.ndim != k.ndim:
            raise ValueError("k and v must both be packed [tokens, heads, dim] or both paged "
                             "[pages, page_size, heads, dim]")
        if k.shape[:-1] != v.shape[:-1]:
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ in more than their head dimension")
        if q.shape[-1] != k.shape[-1]:
            raise ValueError(f"query head dim {q.shape[-1]} differs from key head dim {k.shape[-1]}")
        if not (k.shape[-2] > 0 and q.shape[1] % k.shape[-2] == 0):
            raise ValueError(f"{q.shape[1]} query heads are not a multiple of {k.shape[-2]} key/value heads")
        if not (1 <= q.shape[-1] <= MAX_HEAD_DIM and 1 <= v.shape[-1] <= MAX_HEAD_DIM):
            raise ValueError(f"head dims ({q.shape[-1]}, {v.shape[-1]}) must lie in 1..{MAX_HEAD_DIM}")
        if not (self.cu_q.ndim == 1 and self.cu_q.numel() >= 1):
            raise ValueError("cu_seqlens_q must be a vector of batch + 1 offsets")
        if (self.cu_k is None) == (self.used_k is None):
            raise ValueError("give key lengths exactly once: cu_seqlens_k or seqused_k")
        if (self.table is None) != (k.ndim == 3):
            raise ValueError("paged 4-D K/V goes with a block_table, packed 3-D K/V without one")
        device = q.device
        b, hq, hk = self.batch, self.heads, self.kv_heads
        i32, f32 = (torch.int32,), (torch.float32,)
        _check(self.cu_q, "cu_seqlens_q", (b + 1,), i32, device)
        _check(self.cu_k, "cu_seqlens_k", (b + 1,), i32, device)
        _check(self.used_k, "seqused_k", (b,), i32, device)
        _check(self.table, "block_table", (b, None), i32, device)
        _check(self.leftpad, "leftpad_k", (b,), i32, device)
        _check(self.out, "out", (self.tokens, hq, self.dim_v), (), device)
        window = tuple(self.window)
        if not (len(window) == 2 and min(window) >= -1):
            raise ValueError(f"window_size {window} must be two bounds, each -1 (unbounded) or >= 0")
        if not self.softcap >= 0:
            raise ValueError(f"softcap {self.softcap} must be >= 0 (0 disables it)")
        if not self.splits >= 0:
            raise ValueError(f"num_splits {self.splits} must be >= 0")
        if not (self.max_q >= 0 and self.max_k >= 0):
            raise ValueError(f"max_seqlen_q/max_seqlen_k ({self.max_q}, {self.max_k}) must be >= 0")
        if not (self.mask is None or isinstance(self.mask, MaskSpec)):
            raise TypeError("mask_mod must come from mm_prefix_mask() or rswa_mask()")
        if torch.is_tensor(self.causal):
            _check(self.causal, "dynamic causal flags", (b,), (torch.bool,), device)
        _check(self.q_descale, "q_descale", (b, hk), f32, device)
        _check(self.k_descale, "k_descale", (b, hk), f32, device)
        _check(self.v_descale, "v_descale", (b, hk), f32, device)
        if self.alibi is not None:
            Want("alibi_slopes", {(hq,), (b, hq)}, f32).check(self.alibi, device)
        _check(self.sinks, "s_aux", (hq,), (), device)
        if self.mask is not None:
            if self.mask.kind not in (1, 2) or self.mask_aux is None or len(self.mask_aux) != 2:
                raise ValueError("a vLLM mask needs its two auxiliary tensors")
            if self.mask.kind == 1:
                aux_wants = (Want("mm-prefix ranges", (self.tokens, 2), i32), Want("mm-prefix cu_seqlens", (b + 1,), i32))
            else:
                aux_wants = (Want("rswa prefix lengths", (b,), i32), Want("rswa window", (1,), i32))
            for t, want in zip(self.mask_aux, aux_wants):
                if t is None:
                    raise ValueError(f"{want.name} is missing")
                want.check(t, device)
        elif self.mask_aux is not None:
            raise ValueError("aux_tensors were given without a mask_mod to use them")
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.dtype not in ELEMENT_TYPES:
                raise TypeError(f"{name} is {t.dtype}; attention reads float16, bfloat16, float32 or float8_e4m3fn")
        if self.out is not None and self.out.dtype not in OUTPUT_TYPES:
            raise TypeError(f"out is {self.out.dtype}; outputs are float16, bfloat16 or float32")
        if self.tokens and self.max_q == 1 and not self.deterministic and self.mask is None and self.tokens > b:
            # Single-query rows: at most one per request.
            raise ValueError(f"{self.tokens} query rows for {b} requests with max_seqlen_q=1")
        return self
