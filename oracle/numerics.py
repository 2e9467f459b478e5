"""numpy restatement of the hot-path arithmetic (test infrastructure only).

Every function cites the reference lines it restates (paths relative to
fxeqxmulfx/diff-gpt) and names what pins it (tests/test_oracle.py).

Floating-point conventions:
  * arrays hold float32 values; "bf16"/"f16" tensors are float32 arrays whose
    values are exactly representable in that format (round_to() produces them);
  * float32 numpy arithmetic rounds every operation (no fused multiply-add),
    which is the RoPE / norm contract of the HIP kernels;
  * the float64-model functions (rope_f64, rms_norm_f64) take and return
    float64 arrays.
"""

from __future__ import annotations

import numpy as np

FLT_EPS = np.float32(np.finfo(np.float32).eps)  # F.rms_norm eps=None for fp32 opmath


# ---------------------------------------------------------------------------
# rounding to the storage dtypes
# ---------------------------------------------------------------------------


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 (nearest, ties to even) and return float32.

    Pinned by: known bit patterns (ties, overflow to inf, NaN) and agreement
    with torch.Tensor.to(torch.bfloat16) on random data."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32)
    return (r << 16).astype(np.uint32).view(np.float32)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "f16":
        return f16_round(x)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# RoPE  (rope.py:4-44)
# ---------------------------------------------------------------------------


def freqs_table_f64(dim: int, end: int, theta: float) -> np.ndarray:
    """Exact (float64) RoPE table of rope.py:30-44: [m, j] = (cos m*w_j,
    sin m*w_j), w_j = theta**(-2j/dim).  The product builds its fp32 table with
    torch on the host; this is what that table approximates.

    Pinned by: the reference's known answers test_rope_freqs.py:21-53
    (t=0 -> (1,0); cos(1), sin(1); cos(0.01), sin(0.01)) and unit magnitude."""
    j = np.arange(0, dim, 2, dtype=np.float64)[: dim // 2]
    w = 1.0 / (float(theta) ** (j / dim))
    ang = np.arange(end, dtype=np.float64)[:, None] * w[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1)


def rope(x: np.ndarray, cs: np.ndarray, dtype: str) -> np.ndarray:
    """apply_rotary_emb (rope.py:20-27): interleaved pairs (x[2j], x[2j+1])
    rotated by (cos, sin) = cs[..., j, :] in float32 with separately rounded
    products, rounded once to ``dtype``.

    Pinned by: test_rope.py:14-35 (pi/2 maps (1,0) to (0,1)) and an fp64 2x2
    rotation on random data (the float32 result is within 1 ulp-scale of it)."""
    x = np.asarray(x, dtype=np.float32)
    cs = np.asarray(cs, dtype=np.float32)
    pairs = x.reshape(*x.shape[:-1], -1, 2)
    re, im = pairs[..., 0], pairs[..., 1]
    c, s = cs[..., 0], cs[..., 1]
    out_re = (re * c) - (im * s)
    out_im = (re * s) + (im * c)
    out = np.stack([out_re, out_im], axis=-1).reshape(x.shape)
    return round_to(out, dtype)


# ---------------------------------------------------------------------------
# RMSNorm in the canonical order of the kernels  (rms_norm.py:5-7)
# ---------------------------------------------------------------------------


def tree_sum(v: np.ndarray) -> np.ndarray:
    """Pairwise tree over the last axis, zero-padded to a power of two:
    adjacent pairs, then pairs of pairs ...; every addition rounded in fp32."""
    v = np.asarray(v, dtype=np.float32)
    n = v.shape[-1]
    p = 1
    while p < n:
        p *= 2
    if p != n:
        pad = np.zeros((*v.shape[:-1], p - n), dtype=np.float32)
        v = np.concatenate([v, pad], axis=-1)
    while v.shape[-1] > 1:
        v = v[..., 0::2] + v[..., 1::2]
    return v[..., 0]


def rms_norm(x: np.ndarray, dtype: str) -> np.ndarray:
    """F.rms_norm(x, (N,)) with eps=None: x * 1/sqrt(mean(x^2) + FLT_EPSILON)
    in float32 (bf16/f16 inputs are upcast, rms_norm.py:7), rounded once.
    Order: squares rounded, tree_sum, / N, + eps, correctly rounded sqrt and
    reciprocal, one product.

    Pinned by: torch.nn.functional.rms_norm on the CPU (<= 2 ulp), the closed
    form in fp64, scale invariance and unit RMS (test_rms_norm.py:8-68)."""
    x = np.asarray(x, dtype=np.float32)
    ss = tree_sum(x * x)
    mean = ss / np.float32(x.shape[-1])
    r = np.float32(1.0) / np.sqrt((mean + FLT_EPS).astype(np.float32))
    return round_to(x * r[..., None].astype(np.float32), dtype)


def rope_qknorm(x: np.ndarray, cs: np.ndarray, dtype: str) -> np.ndarray:
    """mha.py:44-48 for one of q / k: rope, round to dtype, then rms_norm."""
    return rms_norm(rope(x, cs, dtype), dtype)


# ---------------------------------------------------------------------------
# float64 models (GPT.double()): rope.py:20-27 and rms_norm.py:5-7 on float64
# ---------------------------------------------------------------------------

DBL_EPS = np.finfo(np.float64).eps  # F.rms_norm eps=None for float64


def rope_f64(x: np.ndarray, cs: np.ndarray) -> np.ndarray:
    """apply_rotary_emb on float64 rows (rope.py:20-27): x.float() rounds x to
    fp32; the products and the sum / difference are evaluated in the promoted
    dtype of fp32 and the table -- float64 for a float64 table (GPT.double()
    converts the buffer), fp32 for an fp32 one -- each operation rounded
    (no fused multiply-add); type_as returns float64 exactly.

    Pinned by: torch's own type promotion of the same expression on the CPU
    for both table dtypes (tests/test_oracle.py), the x.float() rounding on a
    float64 input that fp32 cannot hold, and the quarter turn (1, 0) -> (0, 1)
    of test_rope.py:14-35."""
    ct = np.float64 if np.asarray(cs).dtype == np.float64 else np.float32
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32).astype(ct)
    cs = np.asarray(cs, dtype=ct)
    pairs = x32.reshape(*x32.shape[:-1], -1, 2)
    re, im = pairs[..., 0], pairs[..., 1]
    c, s = cs[..., 0], cs[..., 1]
    out = np.stack([(re * c) - (im * s), (re * s) + (im * c)], axis=-1)
    return out.reshape(x32.shape).astype(np.float64)


def rms_norm_f64(x: np.ndarray) -> np.ndarray:
    """F.rms_norm(x, (N,)) on float64 rows: x / sqrt(mean(x^2) + DBL_EPSILON).
    The summation order is numpy's, so the kernels agree within a few float64
    ulps, not bit for bit.

    Pinned by: torch.nn.functional.rms_norm in float64 on the CPU and unit RMS
    of the result (tests/test_oracle.py)."""
    x = np.asarray(x, dtype=np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + DBL_EPS)


# ---------------------------------------------------------------------------
# attention  (mha.py:61-81)
# ---------------------------------------------------------------------------


def visible_mask(Tq: int, Tk: int) -> np.ndarray:
    """Key j visible to query i: is_causal when Tq == Tk (top-left aligned,
    mha.py:64), everything when Tq == 1 (mha.py:68), otherwise the
    prefix + lower-triangle bool mask of mha.py:69-81."""
    if Tq == Tk:
        return np.tril(np.ones((Tq, Tk), dtype=bool))
    if Tq == 1:
        return np.ones((1, Tk), dtype=bool)
    prefix = Tk - Tq
    m = np.zeros((Tq, Tk), dtype=bool)
    m[:, :prefix] = True
    m[:, prefix:] = np.tril(np.ones((Tq, Tq), dtype=bool))
    return m


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None) -> np.ndarray:
    """softmax(q k^T * scale + mask) v in float64 by brute force.
    q: (B,Tq,H,D); k, v: (B,Tk,H,D) -> (B,Tq,H,D).

    Pinned by: torch.nn.functional.scaled_dot_product_attention (float64, CPU)
    for all three branches, and the one-key / uniform-key closed forms."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    Tq, Tk, D = q.shape[1], k.shape[1], q.shape[3]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    s = np.einsum("bihd,bjhd->bhij", q, k) * scale
    mask = visible_mask(Tq, Tk)
    s = np.where(mask[None, None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("bhij,bjhd->bihd", p, v)


def attention_head_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
                       rows: slice | None = None) -> np.ndarray:
    """attention_f64 for one (row, head): q (Tq, D), k and v (Tk, D) -> (Tq, D),
    as float64 matrix products (BLAS), so sequences of a few thousand keys
    take seconds.  ``rows`` restricts the result to a slice of the queries
    (their mask rows are those of the full Tq x Tk problem).

    Pinned by: equality with attention_f64 within float64 rounding on causal,
    chunked and single-query shapes (tests/test_oracle.py)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    Tq, Tk, D = q.shape[0], k.shape[0], q.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    sel = slice(0, Tq) if rows is None else rows
    s = (q[sel] @ k.T) * scale
    mask = visible_mask(Tq, Tk)[sel]
    s = np.where(mask, s, -np.inf)
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ v


# ---------------------------------------------------------------------------
# KV cache bookkeeping  (kv_cache.py:4-116)
# ---------------------------------------------------------------------------


def grown_capacity(t1: int) -> int:
    """kv_cache.py:92-96.  Pinned by test_kv_cache.py:151-178 (t1 = 21 -> 2048)."""
    return ((t1 + 1024) + 1023) & ~1023


class CacheModel:
    """numpy model of KVCache: (L, 2, B, H, Tcap, D) array, lazy allocation,
    growth, insert at [pos, pos+T), pos advancing after the last layer, and
    batch-broadcast prefill (kv_cache.py:16-116).  Unwritten slots hold NaN so
    a test can tell them apart.

    Pinned by: the fill-value / pos / growth / broadcast known answers of
    test_kv_cache.py:7-227."""

    def __init__(self, B: int, H: int, T: int, D: int, L: int):
        self.shape = (L, 2, B, H, T, D)
        self.data: np.ndarray | None = None
        self.pos = 0

    def insert(self, layer: int, k: np.ndarray, v: np.ndarray):
        """k, v: (B, H, T_add, D)."""
        if self.data is None:
            self.data = np.full(self.shape, np.nan, dtype=np.float32)
        t0, t1 = self.pos, self.pos + k.shape[2]
        if t1 > self.data.shape[4]:
            grown = np.full(
                (*self.data.shape[:4], grown_capacity(t1), self.data.shape[5]),
                np.nan, dtype=np.float32,
            )
            grown[..., : self.data.shape[4], :] = self.data
            self.data = grown
            self.shape = grown.shape
        self.data[layer, 0, :, :, t0:t1] = k
        self.data[layer, 1, :, :, t0:t1] = v
        if layer == self.data.shape[0] - 1:
            self.pos = t1
        return self.data[layer, 0, :, :, :t1], self.data[layer, 1, :, :, :t1]

    def prefill(self, other: "CacheModel"):
        self.data = np.full(self.shape, np.nan, dtype=np.float32)
        n = other.pos
        self.data[..., :n, :] = other.data[..., :n, :]  # broadcasts a batch of 1
        self.pos = n
