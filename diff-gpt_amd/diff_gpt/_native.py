"""Binding of libdgattn.so (the gfx950 HIP library behind include/dgattn.h).

The C entry points are reached through ctypes and exposed to PyTorch as custom
operators in the ``dgattn`` namespace (``torch.ops.dgattn.*``), registered for
the CUDA (= HIP on ROCm) dispatch key only.  There is deliberately no CPU
kernel: a CPU tensor, a missing library or an autograd-tracked input raises
instead of silently computing somewhere else.

Each wrapper passes raw data pointers, element strides and the current HIP
stream of the tensor's device; the library enqueues its kernels on that stream
and returns immediately.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import NamedTuple

import torch

LIB_PATH = Path(
    os.environ.get(
        "DGATTN_LIB", Path(__file__).resolve().parent.parent / "lib" / "libdgattn.so"
    )
)

DG_F32, DG_BF16, DG_F16, DG_F64 = 0, 1, 2, 3
DG_QKNORM = 1
DG_KEYS_NORMED = 2
DG_EUNSUPPORTED = -2
_DTYPE_CODE = {torch.float32: DG_F32, torch.bfloat16: DG_BF16, torch.float16: DG_F16, torch.float64: DG_F64}


class Stride3(ctypes.Structure):
    """``dg_stride3``: element strides of a (B,T,H,D) view."""

    _fields_ = [("b", ctypes.c_int64), ("t", ctypes.c_int64), ("h", ctypes.c_int64)]


class DgPrefix(ctypes.Structure):
    """``dg_prefix``: a prefix shared by groups of rows (see include/dgattn.h)."""

    _fields_ = [("len", ctypes.c_int), ("group", ctypes.c_int), ("k", ctypes.c_void_p),
                ("v", ctypes.c_void_p), ("k_st", Stride3), ("v_st", Stride3), ("own_start", ctypes.c_int)]


class Prefix(NamedTuple):
    """A prefix shared by groups of ``group`` consecutive rows: positions
    0 .. length-1 of every row of a group are the group's.  k, v: the prefix
    pages, (G, length, H, D) views (one entry per group); None when each
    group's first row of the cache holds them.  own_start: the first position
    the per-row cache views hold (length when the prefix lives only in k, v)."""

    length: int
    group: int
    k: torch.Tensor | None = None
    v: torch.Tensor | None = None
    own_start: int = 0


def _prefix_arg(prefix: "Prefix | None"):
    if prefix is None or (prefix.k is None and (prefix.group <= 1 or prefix.length <= 0)):
        return None, 0
    p = DgPrefix()
    p.len, p.group, p.own_start = int(prefix.length), int(prefix.group), int(prefix.own_start)
    if prefix.k is not None:
        p.k, p.v = prefix.k.data_ptr(), prefix.v.data_ptr()
        p.k_st, p.v_st = _bthd_strides(prefix.k), _bthd_strides(prefix.v)
    return ctypes.pointer(p), p.own_start


_lib: ctypes.CDLL | None = None

_SIGNATURES = {
    "dg_abi_version": (ctypes.c_int, []),
    "dg_last_error": (ctypes.c_char_p, []),
    "dg_rope_qknorm_append": (
        ctypes.c_int,
        [ctypes.c_int] * 5
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 7  # q, q_out, k, k_out, v, v_out, freqs
        + [ctypes.c_int, ctypes.c_int, ctypes.c_void_p],
    ),
    "dg_attention_workspace_size": (ctypes.c_size_t, [ctypes.c_int] * 6),
    "dg_attention": (
        ctypes.c_int,
        [ctypes.c_int] * 6
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 4
        + [ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    ),
    "dg_attention_grouped": (
        ctypes.c_int,
        [ctypes.c_int] * 6
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 4
        + [ctypes.c_float, ctypes.POINTER(DgPrefix), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    ),
    "dg_lm_head": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_void_p],
    ),
    "dg_prefill_rope": (
        ctypes.c_int,
        [ctypes.c_int] * 6
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 2  # q, freqs
        + [ctypes.c_int, ctypes.c_int]  # freqs dtype, flags
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 3  # k, v, y
        + [ctypes.c_float, ctypes.c_void_p],
    ),
    "dg_rope_qknorm_append_at": (
        ctypes.c_int,
        [ctypes.c_int] * 4
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 6  # q, q_out, k, k_cache, v, v_cache
        + [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
           ctypes.c_int, ctypes.c_void_p],
    ),
    "dg_decode_attention_at_workspace_size": (ctypes.c_size_t, [ctypes.c_int] * 5),
    "dg_decode_attention_at": (
        ctypes.c_int,
        [ctypes.c_int] * 4
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 4  # q, k_cache, v_cache, y
        + [ctypes.c_float, ctypes.POINTER(DgPrefix), ctypes.c_void_p, ctypes.c_int,
           ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    ),
    "dg_decode_step_workspace_size": (ctypes.c_size_t, [ctypes.c_int] * 5),
    "dg_decode_step": (
        ctypes.c_int,
        [ctypes.c_int] * 4
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 5  # q, k, v, k_cache, v_cache
        + [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        + [ctypes.c_void_p, ctypes.POINTER(Stride3), ctypes.c_float, ctypes.POINTER(DgPrefix),
           ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    ),
    "dg_decode_step_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "dg_decode_step_noalloc": (
        ctypes.c_int,
        [ctypes.c_int] * 4
        + [ctypes.c_void_p, ctypes.POINTER(Stride3)] * 5  # q, k, v, k_cache, v_cache
        + [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        + [ctypes.c_void_p, ctypes.POINTER(Stride3), ctypes.c_float, ctypes.POINTER(DgPrefix),
           ctypes.c_int, ctypes.c_void_p],
    ),
    "dg_rms_norm": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p],
    ),
    "dg_embed_norm": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p],
    ),
    "dg_copy4d": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p,
         ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64),
         ctypes.c_void_p],
    ),
    "dg_attn_res_norm": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
         ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_void_p],
    ),
    "dg_gate": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p],
    ),
    "dg_swiglu": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_double, ctypes.c_double, ctypes.c_void_p],
    ),
    "dg_softcap": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_double, ctypes.c_void_p],
    ),
    "dg_block_out": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
         ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_float, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p],
    ),
    "dg_draw_argmax": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p],
    ),
    "dg_block_out_norm": (
        ctypes.c_int,
        [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
         ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_float, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p],
    ),
}

ABI_VERSION = 3

# head_dim the kernels take: every even size up to 1024 (a row padded to the
# next power of two spreads over at most 64 lanes of 16 elements)
MAX_HEAD_DIM = 1024


def head_dim_supported(D: int) -> bool:
    """Whether every kernel of the attention path takes this head_dim."""
    return 2 <= D <= MAX_HEAD_DIM and D % 2 == 0


def lib() -> ctypes.CDLL:
    """Load libdgattn.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"libdgattn.so not found at {LIB_PATH}; build it with "
                "`python diff-gpt_amd/csrc/build.py` (or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        got = handle.dg_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"libdgattn ABI {got} != expected {ABI_VERSION}")
        _lib = handle
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().dg_last_error().decode(errors="replace")
        raise RuntimeError(f"dgattn.{what} failed (status {rc}): {msg}")


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(
            f"dgattn supports float32/bfloat16/float16/float64 tensors, got {t.dtype}"
        ) from None


def require_device(what: str, *tensors: torch.Tensor | None) -> None:
    """The HIP path has no CPU implementation: insist on ROCm device tensors."""
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{what}: the MI355X attention path runs on ROCm devices only; got a "
                f"tensor on '{t.device}'. Move the model/cache with .to('cuda')."
            )


def require_device_type(what: str, device) -> None:
    if torch.device(device).type != "cuda":
        raise RuntimeError(
            f"{what}: the MI355X attention path runs on ROCm devices only; got '{device}'"
        )


def require_inference(what: str, *tensors: torch.Tensor | None) -> None:
    if not torch.is_grad_enabled():
        return
    for t in tensors:
        if t is not None and t.requires_grad:
            raise RuntimeError(
                f"{what}: the HIP kernels are inference-only (no backward); call under "
                "torch.no_grad() / torch.inference_mode()"
            )


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _bthd_strides(t: torch.Tensor) -> Stride3:
    """Strides of a 4-D (B,T,H,D) view with a unit D stride."""
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D (B,T,H,D) tensor, got shape {tuple(t.shape)}")
    if t.stride(3) != 1 and t.size(3) > 1:
        raise ValueError("the last (head_dim) dimension must be contiguous")
    return Stride3(t.stride(0), t.stride(1), t.stride(2))


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


# ---------------------------------------------------------------------------
# Raw launchers (operate in place on caller-provided outputs)
# ---------------------------------------------------------------------------


def rope_qknorm_append_(
    q: torch.Tensor | None,
    k: torch.Tensor | None,
    v: torch.Tensor | None,
    freqs: torch.Tensor,
    q_out: torch.Tensor | None,
    k_out: torch.Tensor | None,
    v_out: torch.Tensor | None,
    qknorm: bool,
) -> None:
    """dg_rope_qknorm_append on (B,T,H,D) views; freqs is (B|1,T,H|1,D/2,2)."""
    ref = next(t for t in (q, k, v) if t is not None)
    B, T, H, D = ref.shape
    for a, b in ((q, q_out), (k, k_out), (v, v_out)):
        if (a is None) != (b is None):
            raise ValueError("each input needs an output (and vice versa)")
        if a is not None:
            if a.shape != (B, T, H, D) or b.shape != (B, T, H, D):
                raise ValueError(f"shape mismatch: {tuple(a.shape)} -> {tuple(b.shape)}")
            if a.dtype != ref.dtype or b.dtype != ref.dtype:
                raise TypeError("q/k/v and outputs must share one dtype")
    need_f = q is not None or k is not None
    if need_f:
        if freqs.dim() != 5 or freqs.shape[-2:] != (D // 2, 2):
            raise ValueError(f"freqs must be (B,T,H,D/2,2)-broadcastable, got {tuple(freqs.shape)}")
        if freqs.stride(-1) != 1 or freqs.stride(-2) != 2:
            freqs = freqs.contiguous()
        if freqs.size(1) not in (1, T) or freqs.size(0) not in (1, B) or freqs.size(2) not in (1, H):
            raise ValueError("freqs does not broadcast against (B,T,H)")
        fb = 0 if freqs.size(0) == 1 else freqs.stride(0)
        ft = 0 if freqs.size(1) == 1 else freqs.stride(1)
        fh = 0 if freqs.size(2) == 1 else freqs.stride(2)
        f_st = Stride3(fb, ft, fh)
        f_code = _dtype_code(freqs)
    else:
        f_st = Stride3(0, 0, 0)
        f_code = _dtype_code(ref)

    def st(t):
        return None if t is None else ctypes.pointer(_bthd_strides(t))

    rc = lib().dg_rope_qknorm_append(
        B, T, H, D, _dtype_code(ref),
        _ptr(q), st(q), _ptr(q_out), st(q_out),
        _ptr(k), st(k), _ptr(k_out), st(k_out),
        _ptr(v), st(v), _ptr(v_out), st(v_out),
        _ptr(freqs if need_f else None), ctypes.pointer(f_st), f_code,
        DG_QKNORM if qknorm else 0, _stream(ref),
    )
    _check(rc, "rope_qknorm_append")


def attention_(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, y: torch.Tensor,
               scale: float, prefix_len: int = 0, group: int = 1, prefix: Prefix | None = None) -> None:
    """dg_attention_grouped: q,y (B,Tq,H,D) views; k,v (B,Tk - own_start,H,D)
    views of the rows' keys from position own_start on.  With group > 1 the
    first prefix_len keys of row b are read from row (b // group) * group (rows
    of a group must hold identical prefixes); ``prefix`` (a Prefix) names
    separate prefix pages instead."""
    if prefix is None:
        prefix = Prefix(prefix_len, group)
    parg, own_start = _prefix_arg(prefix)
    B, Tq, H, D = q.shape
    Tk = k.size(1) + own_start
    if k.shape != (B, Tk - own_start, H, D) or v.shape != k.shape or y.shape != q.shape:
        raise ValueError("attention: inconsistent q/k/v/y shapes")
    if not (q.dtype == k.dtype == v.dtype == y.dtype):
        raise TypeError("attention: q/k/v/y must share one dtype")
    code = _dtype_code(q)
    L = lib()
    ws_bytes = L.dg_attention_workspace_size(B, H, Tq, Tk, D, code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    rc = L.dg_attention_grouped(
        B, H, Tq, Tk, D, code,
        _ptr(q), ctypes.pointer(_bthd_strides(q)),
        _ptr(k), ctypes.pointer(_bthd_strides(k)),
        _ptr(v), ctypes.pointer(_bthd_strides(v)),
        _ptr(y), ctypes.pointer(_bthd_strides(y)),
        float(scale), parg, _ptr(ws), ws_bytes, _stream(q),
    )
    _check(rc, "attention")


def prefill_rope_(q: torch.Tensor, freqs: torch.Tensor, k: torch.Tensor, v: torch.Tensor, y: torch.Tensor,
                  scale: float, qknorm: bool, keys_normed: bool = False) -> bool:
    """dg_prefill_rope: attention over k, v (B,Tk,H,D) views of the query rows
    q (B,Tq,H,D) after RoPE (freqs (B|1,Tq,H|1,D/2,2)) and, with qknorm, the
    QK-norm -- applied as the kernel loads q -- into y.  keys_normed (with
    qknorm) declares every key row RMS-normalised, which bounds the scores and
    lets the kernel drop the softmax's running maximum.  Returns False, having
    done nothing, when the fused kernel does not take the shape (the caller
    then makes the two calls); raises on any other error."""
    B, Tq, H, D = q.shape
    Tk = k.size(1)
    if k.shape != (B, Tk, H, D) or v.shape != (B, Tk, H, D) or y.shape != q.shape:
        raise ValueError("prefill_rope: inconsistent q/k/v/y shapes")
    if not (q.dtype == k.dtype == v.dtype == y.dtype):
        raise TypeError("prefill_rope: q/k/v/y must share one dtype")
    if freqs.dim() != 5 or freqs.shape[-2:] != (D // 2, 2):
        raise ValueError(f"freqs must be (B,T,H,D/2,2)-broadcastable, got {tuple(freqs.shape)}")
    if freqs.stride(-1) != 1 or freqs.stride(-2) != 2:
        freqs = freqs.contiguous()
    if freqs.size(1) not in (1, Tq) or freqs.size(0) not in (1, B) or freqs.size(2) not in (1, H):
        raise ValueError("freqs does not broadcast against (B,Tq,H)")
    f_st = Stride3(*(0 if freqs.size(i) == 1 else freqs.stride(i) for i in range(3)))
    st = lambda t: ctypes.pointer(_bthd_strides(t))  # noqa: E731
    rc = lib().dg_prefill_rope(
        B, H, Tq, Tk, D, _dtype_code(q), _ptr(q), st(q), _ptr(freqs), ctypes.pointer(f_st), _dtype_code(freqs),
        (DG_QKNORM if qknorm else 0) | (DG_KEYS_NORMED if qknorm and keys_normed else 0),
        _ptr(k), st(k), _ptr(v), st(v), _ptr(y), st(y), float(scale), _stream(q),
    )
    if rc == DG_EUNSUPPORTED:
        return False
    _check(rc, "prefill_rope")
    return True


def lm_head_(x: torch.Tensor, w: torch.Tensor, cap: float, logits: torch.Tensor,
             ids: torch.Tensor | None = None) -> bool:
    """dg_lm_head: logits (M, V) = softcap(x (M, C) @ w (V, C)^T) with cap
    (0 = none), and with ids (M,) int64 the first maximum of every logits row.
    Returns False, having done nothing, when the fused kernel does not take the
    shape (the caller then runs F.linear + softcap + argmax)."""
    M, C = x.shape
    V = w.size(0)
    if w.shape != (V, C) or logits.shape != (M, V):
        raise ValueError("lm_head: inconsistent x/w/logits shapes")
    if not (x.dtype == w.dtype == logits.dtype):
        raise TypeError("lm_head: x, w and logits must share one dtype")
    if x.stride(1) != 1 or w.stride(1) != 1 or logits.stride(1) != 1:
        return False
    if ids is not None and (ids.shape != (M,) or ids.dtype != torch.int64 or not ids.is_contiguous()):
        raise ValueError("lm_head: ids must be a contiguous (M,) int64 tensor")
    rc = lib().dg_lm_head(
        M, C, V, _dtype_code(x), _ptr(x), x.stride(0), _ptr(w), w.stride(0), float(cap),
        _ptr(logits), logits.stride(0), _ptr(ids), _stream(x),
    )
    if rc == DG_EUNSUPPORTED:
        return False
    _check(rc, "lm_head")
    return True


def rope_qknorm_append_at_(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    freqs_table: torch.Tensor,
    q_out: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    pos: torch.Tensor,
    qknorm: bool,
) -> None:
    """dg_rope_qknorm_append_at: q, k, v, q_out (B,1,H,D); k_cache / v_cache the
    (B,Tcap,H,D) cache views at position 0; freqs_table (Tmax, D/2, 2); pos a
    one-element int32 device tensor (positions already cached)."""
    B, T, H, D = q.shape
    if T != 1 or k.shape != q.shape or v.shape != q.shape or q_out.shape != q.shape:
        raise ValueError("rope_qknorm_append_at: q, k, v, q_out must be (B, 1, H, D)")
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[2:] != (H, D):
        raise ValueError("rope_qknorm_append_at: cache views must be (B, Tcap, H, D)")
    if v_cache.shape != k_cache.shape:
        raise ValueError("rope_qknorm_append_at: k and v caches differ in shape")
    if freqs_table.dim() != 3 or freqs_table.shape[1:] != (D // 2, 2) or not freqs_table.is_contiguous():
        raise ValueError("rope_qknorm_append_at: freqs_table must be a contiguous (Tmax, D/2, 2) table")
    if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != q.device:
        raise TypeError("rope_qknorm_append_at: pos must be a one-element int32 tensor on q's device")
    max_pos = min(k_cache.size(1), freqs_table.size(0))
    st = lambda t: ctypes.pointer(_bthd_strides(t))  # noqa: E731
    rc = lib().dg_rope_qknorm_append_at(
        B, H, D, _dtype_code(q),
        _ptr(q), st(q), _ptr(q_out), st(q_out),
        _ptr(k), st(k), _ptr(k_cache), st(k_cache),
        _ptr(v), st(v), _ptr(v_cache), st(v_cache),
        _ptr(freqs_table), freqs_table.stride(0), _dtype_code(freqs_table),
        _ptr(pos), max_pos, DG_QKNORM if qknorm else 0, _stream(q),
    )
    _check(rc, "rope_qknorm_append_at")


def decode_attention_at_(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    y: torch.Tensor,
    scale: float,
    pos: torch.Tensor,
    prefix_len: int = 0,
    group: int = 1,
    prefix: Prefix | None = None,
) -> None:
    """dg_decode_attention_at: q, y (B,1,H,D); k_cache / v_cache (B,Tcap,H,D)
    views from position own_start; attends over positions 0 .. pos[0]."""
    if prefix is None:
        prefix = Prefix(prefix_len, group)
    parg, own_start = _prefix_arg(prefix)
    B, T, H, D = q.shape
    if T != 1 or y.shape != q.shape:
        raise ValueError("decode_attention_at: q and y must be (B, 1, H, D)")
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[2:] != (H, D) or v_cache.shape != k_cache.shape:
        raise ValueError("decode_attention_at: cache views must be (B, Tcap, H, D)")
    if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != q.device:
        raise TypeError("decode_attention_at: pos must be a one-element int32 tensor on q's device")
    code = _dtype_code(q)
    L = lib()
    max_keys = k_cache.size(1) + own_start
    ws_bytes = L.dg_decode_attention_at_workspace_size(B, H, max_keys, D, code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    st = lambda t: ctypes.pointer(_bthd_strides(t))  # noqa: E731
    rc = L.dg_decode_attention_at(
        B, H, D, code, _ptr(q), st(q), _ptr(k_cache), st(k_cache), _ptr(v_cache), st(v_cache),
        _ptr(y), st(y), float(scale), parg, _ptr(pos), max_keys,
        _ptr(ws), ws_bytes, _stream(q),
    )
    _check(rc, "decode_attention_at")


def decode_step_(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    freqs: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    y: torch.Tensor,
    scale: float,
    pos: int | torch.Tensor,
    prefix_len: int = 0,
    group: int = 1,
    qknorm: bool = True,
    noalloc: bool = False,
    prefix: Prefix | None = None,
) -> None:
    """dg_decode_step: RoPE + QK-norm of the step's q, k (B,1,H,D), the K/V
    append at position p of the (B,Tcap,H,D) cache views (at position 0), and
    the decode attention over positions 0 .. p into y (B,1,H,D).  pos is p as a
    Python int, with freqs the (D/2, 2) (cos, sin) row of position p; or a
    one-element int32 device tensor holding p, with freqs the whole contiguous
    (Tmax, D/2, 2) table.  noalloc=True calls dg_decode_step_noalloc, whose
    key-split partials live in the library's static device scratch instead of
    a workspace allocated here.  ``prefix`` (a Prefix) replaces prefix_len /
    group; with own_start > 0 the cache views hold positions own_start on."""
    if prefix is None:
        prefix = Prefix(prefix_len, group)
    parg, own_start = _prefix_arg(prefix)
    B, T, H, D = q.shape
    if T != 1 or k.shape != q.shape or v.shape != q.shape or y.shape != q.shape:
        raise ValueError("decode_step: q, k, v, y must be (B, 1, H, D)")
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[2:] != (H, D) or v_cache.shape != k_cache.shape:
        raise ValueError("decode_step: cache views must be (B, Tcap, H, D)")
    max_pos = k_cache.size(1) + own_start
    if isinstance(pos, torch.Tensor):
        if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != q.device:
            raise TypeError("decode_step: a device position must be a one-element int32 tensor on q's device")
        if freqs.dim() != 3 or freqs.shape[1:] != (D // 2, 2) or not freqs.is_contiguous():
            raise ValueError("decode_step: with a device position freqs must be the contiguous (Tmax, D/2, 2) table")
        fstride, pos_host, pos_ptr = freqs.stride(0), 0, _ptr(pos)
        max_pos = min(max_pos, freqs.size(0))
    else:
        if freqs.numel() != D or not freqs.is_contiguous():
            raise ValueError("decode_step: with a host position freqs must be the contiguous (cos, sin) row of it")
        fstride, pos_host, pos_ptr = 0, int(pos), None
    code = _dtype_code(q)
    L = lib()
    st = lambda t: ctypes.pointer(_bthd_strides(t))  # noqa: E731
    args = (
        B, H, D, code, _ptr(q), st(q), _ptr(k), st(k), _ptr(v), st(v),
        _ptr(k_cache), st(k_cache), _ptr(v_cache), st(v_cache),
        _ptr(freqs), fstride, _dtype_code(freqs), pos_host, pos_ptr, max_pos,
        _ptr(y), st(y), float(scale), parg, DG_QKNORM if qknorm else 0,
    )
    if noalloc:
        _check(L.dg_decode_step_noalloc(*args, _stream(q)), "decode_step_noalloc")
        return
    ws_bytes = L.dg_decode_step_workspace_size(B, H, max_pos, D, code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    _check(L.dg_decode_step(*args, _ptr(ws), ws_bytes, _stream(q)), "decode_step")


def rms_norm_(x: torch.Tensor, out: torch.Tensor) -> None:
    N = x.size(-1)
    x2 = x.reshape(-1, N) if x.dim() != 2 else x
    o2 = out.view(-1, N)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    rc = lib().dg_rms_norm(
        x2.size(0), N, _dtype_code(x2), _ptr(x2), x2.stride(0), _ptr(o2), o2.stride(0), _stream(x2)
    )
    _check(rc, "rms_norm")


def embed_norm_(ids: torch.Tensor, table: torch.Tensor, x_out: torch.Tensor,
                xn_out: torch.Tensor | None) -> bool:
    """x_out = rms_norm(table[ids]) and, when given, xn_out = rms_norm(x_out)
    in one dg_embed_norm launch (bits of the separate launches; ids outside
    the table give NaN rows).  False, with nothing launched, for what it does
    not take: fp64, C > 8192, a table or output without unit column stride."""
    V, C = table.shape
    if table.dtype not in (torch.float32, torch.bfloat16, torch.float16) or C > 8192:
        return False
    if table.stride(1) != 1 or ids.dtype != torch.int64:
        return False
    outs = [x_out] if xn_out is None else [x_out, xn_out]
    o2 = []
    for o in outs:
        if o.dtype != table.dtype or not o.is_contiguous() or o.numel() != ids.numel() * C:
            return False
        o2.append(o.view(-1, C))
    i1 = ids.reshape(-1)
    if not i1.is_contiguous():
        i1 = i1.contiguous()
    xn2 = o2[1] if xn_out is not None else None
    rc = lib().dg_embed_norm(
        i1.numel(), C, _dtype_code(table), _ptr(i1), V, _ptr(table), table.stride(0),
        _ptr(o2[0]), C, _ptr(xn2), C, _stream(table),
    )
    _check(rc, "embed_norm")
    return True


def draw_argmax_(probs: torch.Tensor, q: torch.Tensor, ids: torch.Tensor) -> bool:
    """ids (..., 1) int64 = torch.argmax(probs / q, dim=-1, keepdim=True) in one
    dg_draw_argmax launch.  False, with nothing launched, for operands it
    does not take (rows without unit column stride, mixed dtypes)."""
    V = probs.size(-1)
    if q.shape != probs.shape or q.dtype != probs.dtype or probs.dtype not in _DTYPE_CODE:
        return False
    if ids.dtype != torch.int64 or not ids.is_contiguous() or ids.numel() * V != probs.numel():
        return False
    p2, q2 = probs.reshape(-1, V), q.reshape(-1, V)
    if p2.stride(-1) != 1 or q2.stride(-1) != 1:
        return False
    rc = lib().dg_draw_argmax(p2.size(0), V, _dtype_code(p2), _ptr(p2), p2.stride(0), _ptr(q2), q2.stride(0),
                              _ptr(ids), _stream(p2))
    _check(rc, "draw_argmax")
    return True


def copy4d_(src: torch.Tensor, dst: torch.Tensor) -> None:
    """dst[...] = src[...] over 4-D views (src may broadcast with 0 strides)."""
    if src.dim() != 4 or dst.dim() != 4:
        raise ValueError("copy4d expects 4-D views")
    if src.dtype != dst.dtype:
        raise TypeError("copy4d: dtype mismatch")
    shape = (ctypes.c_int64 * 4)(*dst.shape)
    s_st = (ctypes.c_int64 * 4)(*[0 if src.size(i) == 1 and dst.size(i) != 1 else src.stride(i)
                                  for i in range(4)])
    d_st = (ctypes.c_int64 * 4)(*dst.stride())
    for i in range(4):
        if src.size(i) not in (1, dst.size(i)):
            raise ValueError(f"copy4d: {tuple(src.shape)} does not broadcast to {tuple(dst.shape)}")
    rc = lib().dg_copy4d(_dtype_code(dst), shape, _ptr(src), s_st, _ptr(dst), d_st, _stream(dst))
    _check(rc, "copy4d")


def _rows(x: torch.Tensor, what: str) -> torch.Tensor:
    """(..., N) as a 2-D (M, N) view with unit column stride (a copy only when
    the leading dims cannot be merged)."""
    x2 = x.reshape(-1, x.size(-1))
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def attn_res_norm_(sources: list[torch.Tensor], w: torch.Tensor, out: torch.Tensor) -> None:
    """out = rms_norm(block_attn_res(sources[:-1], sources[-1], w)) row by row."""
    C = out.size(-1)
    n = len(sources)
    srcs = [_rows(t, "attn_res_norm") for t in sources]
    for t in srcs:
        if t.shape != srcs[0].shape or t.dtype != out.dtype:
            raise ValueError("attn_res_norm: sources must share shape and dtype with the output")
    o2 = out.view(-1, C)
    w1 = w.reshape(-1).contiguous()
    ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in srcs])
    lds = (ctypes.c_int64 * n)(*[t.stride(0) for t in srcs])
    rc = lib().dg_attn_res_norm(
        o2.size(0), C, _dtype_code(o2), n, ptrs, lds, _ptr(w1), _ptr(o2), o2.stride(0), _stream(o2)
    )
    _check(rc, "attn_res_norm")


def _row_list(tensors: list[torch.Tensor], what: str):
    rows = [_rows(t, what) for t in tensors]
    ptrs = (ctypes.c_void_p * max(1, len(rows)))(*[t.data_ptr() for t in rows])
    lds = (ctypes.c_int64 * max(1, len(rows)))(*[t.stride(0) for t in rows])
    return rows, ptrs, lds


def block_out_(y: torch.Tensor, g: torch.Tensor, w_proj: torch.Tensor, partial_in: torch.Tensor | None,
               blocks: list[torch.Tensor], w_mix: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
               alpha: float, limit: float, out: torch.Tensor, xn_out: torch.Tensor | None = None) -> bool:
    """dg_block_out: from the attention output y (..., C) and the gate logits
    g, the layer's new partial sum into out: c_proj(y * sigmoid(g)), added to
    partial_in unless that is None (the layer commits its input), then plus
    the FFN of the MLP mixture over blocks and that partial.  With xn_out
    (dg_block_out_norm) also rms_norm(out) into it.  Returns False, having
    done nothing, for shapes the fused kernel does not take."""
    C = out.size(-1)
    y2, g2, o2 = _rows(y, "block_out"), _rows(g, "block_out"), out.view(-1, C)
    p2 = None if partial_in is None else _rows(partial_in, "block_out")
    _, ptrs, lds = _row_list(blocks, "block_out")
    ws = (w_proj, w_up, w_down)
    if any(t.stride(1) != 1 or t.dtype != out.dtype for t in ws) or o2.stride(1) != 1:
        return False
    x2 = None
    if xn_out is not None:
        if xn_out.dtype != out.dtype or xn_out.shape != out.shape or not xn_out.is_contiguous():
            return False
        x2 = xn_out.view(-1, C)
    args = [
        o2.size(0), C, _dtype_code(o2), _ptr(y2), y2.stride(0), _ptr(g2), g2.stride(0), _ptr(w_proj),
        w_proj.stride(0), _ptr(p2), 0 if p2 is None else p2.stride(0), len(blocks), ptrs, lds,
        _ptr(w_mix.reshape(-1).contiguous()), _ptr(w_up), w_up.stride(0), _ptr(w_down), w_down.stride(0),
        float(alpha), float(limit), _ptr(o2), o2.stride(0),
    ]
    if x2 is None:
        rc = lib().dg_block_out(*args, _stream(o2))
    else:
        rc = lib().dg_block_out_norm(*args, _ptr(x2), C, _stream(o2))
    if rc == DG_EUNSUPPORTED:
        return False
    _check(rc, "block_out")
    return True


def gate_(y: torch.Tensor, g: torch.Tensor) -> None:
    """y <- y * sigmoid(g), in place."""
    C = y.size(-1)
    y2, g2 = y.view(-1, C), _rows(g, "gate")
    rc = lib().dg_gate(y2.size(0), C, _dtype_code(y2), _ptr(y2), y2.stride(0), _ptr(g2), g2.stride(0),
                       _ptr(y2), y2.stride(0), _stream(y2))
    _check(rc, "gate")


def swiglu_(x: torch.Tensor, out: torch.Tensor, alpha: float, limit: float) -> None:
    N = out.size(-1)
    x2, o2 = _rows(x, "swiglu"), out.view(-1, N)
    rc = lib().dg_swiglu(x2.size(0), N, _dtype_code(x2), _ptr(x2), x2.stride(0), _ptr(o2), o2.stride(0),
                         float(alpha), float(limit), _stream(x2))
    _check(rc, "swiglu")


def softcap_(x: torch.Tensor, cap: float) -> None:
    """x <- cap * tanh(x / cap), in place."""
    N = x.size(-1)
    x2 = x.view(-1, N)
    rc = lib().dg_softcap(x2.size(0), N, _dtype_code(x2), _ptr(x2), x2.stride(0), _ptr(x2), x2.stride(0),
                          float(cap), _stream(x2))
    _check(rc, "softcap")


# ---------------------------------------------------------------------------
# torch.ops.dgattn registration (CUDA/HIP kernels + Meta shape functions)
# ---------------------------------------------------------------------------

_DEF = torch.library.Library("dgattn", "DEF")
_DEF.define(
    "rope_qknorm_append(Tensor? q, Tensor? k, Tensor? v, Tensor freqs, Tensor(a!)? q_out, "
    "Tensor(b!)? k_out, Tensor(c!)? v_out, bool qknorm) -> ()"
)
_DEF.define(
    "attention(Tensor q, Tensor k, Tensor v, float scale, int prefix_len=0, int group=1) -> Tensor"
)
_DEF.define("rms_norm(Tensor x) -> Tensor")
_DEF.define("rope(Tensor x, Tensor freqs) -> Tensor")
_DEF.define("copy4d(Tensor src, Tensor(a!) dst) -> ()")
_DEF.define("attn_res_norm(Tensor[] sources, Tensor w) -> Tensor")
_DEF.define("gate_(Tensor(a!) y, Tensor g) -> ()")
_DEF.define("swiglu(Tensor x, float alpha, float limit) -> Tensor")
_DEF.define("softcap_(Tensor(a!) x, float cap) -> ()")

_IMPL = torch.library.Library("dgattn", "IMPL")


def _attention_impl(q, k, v, scale, prefix_len=0, group=1):
    y = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    attention_(q, k, v, y, scale, prefix_len, group)
    return y


def _rms_norm_impl(x):
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rms_norm_(x, out)
    return out


def _rope_impl(x, freqs):
    # x (..., D) and freqs (..., D/2, 2) broadcast over the leading dims; the
    # kernel sees both as (B,T,H,D) views.
    D = x.size(-1)
    lead = torch.broadcast_shapes(x.shape[:-1], freqs.shape[:-2])
    if tuple(lead) != tuple(x.shape[:-1]):
        raise ValueError("apply_rotary_emb: freqs broadcasts x to a larger shape")
    n = len(lead)
    fexp = freqs.expand(*lead, D // 2, 2)  # 0-stride view over broadcast dims
    if n <= 3:
        pad = (1,) * (3 - n)
        x4 = x.reshape(*pad, *x.shape)
        f5 = fexp.reshape(*pad, *fexp.shape)
    else:
        head = math.prod(lead[:-2])
        x4 = x.reshape(head, *x.shape[-3:])
        f5 = fexp.reshape(head, *lead[-2:], D // 2, 2)
    out = torch.empty(x4.shape, dtype=x.dtype, device=x.device)
    rope_qknorm_append_(x4, None, None, f5, out, None, None, qknorm=False)
    return out.view(x.shape)


def _attn_res_norm_impl(sources, w):
    out = torch.empty(sources[-1].shape, dtype=sources[-1].dtype, device=sources[-1].device)
    attn_res_norm_(list(sources), w, out)
    return out


def _swiglu_impl(x, alpha, limit):
    out = torch.empty((*x.shape[:-1], x.size(-1) // 2), dtype=x.dtype, device=x.device)
    swiglu_(x, out, alpha, limit)
    return out


_IMPL.impl("attn_res_norm", _attn_res_norm_impl, "CUDA")
_IMPL.impl("gate_", gate_, "CUDA")
_IMPL.impl("swiglu", _swiglu_impl, "CUDA")
_IMPL.impl("softcap_", softcap_, "CUDA")
_IMPL.impl("attn_res_norm", lambda sources, w: torch.empty_like(sources[-1]), "Meta")
_IMPL.impl(
    "swiglu", lambda x, alpha, limit: x.new_empty((*x.shape[:-1], x.size(-1) // 2)), "Meta"
)
_IMPL.impl("rope_qknorm_append", rope_qknorm_append_, "CUDA")
_IMPL.impl("attention", _attention_impl, "CUDA")
_IMPL.impl("rms_norm", _rms_norm_impl, "CUDA")
_IMPL.impl("rope", _rope_impl, "CUDA")
_IMPL.impl("copy4d", copy4d_, "CUDA")

_IMPL.impl("attention", lambda q, k, v, scale, prefix_len=0, group=1: torch.empty_like(q), "Meta")
_IMPL.impl("rms_norm", lambda x: torch.empty_like(x), "Meta")
_IMPL.impl("rope", lambda x, freqs: torch.empty_like(x), "Meta")


def ops():
    """The registered operator namespace (torch.ops.dgattn)."""
    return torch.ops.dgattn
