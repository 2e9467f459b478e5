"""Sigma-delta tokenizer of the forecasting API (src/diff_gpt/encoder_decoder.py:1-427).

Host-side arithmetic that turns a multivariate series (T rows x F columns)
into integer tokens in [0, vocab_size) and back.  Every column is first
differenced k times (k = order_of_derivative, per column or shared), scaled
so that the column's domain of definition fits the vocabulary, and quantised
with noise shaping, so that the k-fold integration at decode time does not
accumulate rounding error:

  * k <= 1, or a vocabulary too small for the cascade: a carry scheme -- the
    integer part of each value plus the rounded running sum of the fractional
    parts, differenced;
  * k >= 2 with vocab_size > 2^k + 2: a k-stage MASH sigma-delta cascade whose
    stage outputs are recombined through binomial difference filters, which
    keeps |decoded - input| bounded independently of the series length;
  * k == 0 in the per-column path: plain rounding.

The arithmetic is float64 numpy, or Python Decimal objects in numpy object
arrays (use_decimal=True) for high orders where float64 loses bits in the
k-fold cumulative sums.  The operations are applied in the reference's order
so that the tokens are the same bit for bit (checked against the reference's
outputs in tests/golden/codec.json).  Not accelerated: it runs once per
forecast on a few hundred values, outside the attention hot path.
"""

from __future__ import annotations

import math
from decimal import Decimal

import numpy as np

_decimal_of = np.frompyfunc(Decimal, 1, 1)
_round_obj = np.frompyfunc(round, 1, 1)  # Decimal -> int, ties to even


def np_to_decimal(inp: np.ndarray) -> np.ndarray:
    """Element-wise Decimal(x) of a float array (object array; a 0-d input
    gives a 0-d object array)."""
    out = _decimal_of(inp)
    return np.array(out) if isinstance(out, Decimal) else out


def np_is_decimal(inp: np.ndarray) -> bool:
    if inp.ndim == 0 or inp.shape[0] == 0:
        return inp.dtype == "object"
    first = inp[0] if inp.ndim == 1 else inp[0, 0]
    return isinstance(first, Decimal)


def np_is_float64(inp: np.ndarray) -> bool:
    return inp.dtype == np.dtype("float64")


def _is_scalar_order(order_of_derivative) -> bool:
    return isinstance(order_of_derivative, (int, np.integer))


def _check_kind(x: np.ndarray, use_decimal: bool) -> None:
    if use_decimal:
        assert np_is_decimal(x)
    else:
        assert np_is_float64(x)


def _zeros(shape, like_decimal: bool, dtype=np.float64) -> np.ndarray:
    z = np.zeros(shape, dtype=dtype)
    return np_to_decimal(z) if like_decimal else z


def _uses_cascade(k: int, vocab_size: int) -> bool:
    """MASH needs headroom 2^k in the vocabulary (encoder_decoder.py:244, :321)."""
    return k >= 2 and vocab_size > 2**k + 2


# ---------------------------------------------------------------------------
# k-th differences and their inverse (encoder_decoder.py:36-152)
# ---------------------------------------------------------------------------


def differentiate(
    inp: np.ndarray, order_of_derivative: int | np.ndarray, use_decimal: bool
) -> tuple[np.ndarray, np.ndarray]:
    """Returns (start, diff).

    Shared k: start stacks the first row of each of the k difference levels
    (level 0 = the input), diff is the k-th difference, (T - k, F).
    Per-column k: start is the raw prefix inp[:max_k], and column c of diff is
    the k_c-th difference trimmed to the common length T - max_k."""
    if _is_scalar_order(order_of_derivative):
        k = int(order_of_derivative)
        assert 0 <= k <= inp.shape[0]
        _check_kind(inp, use_decimal)
        level = inp
        heads = []
        for _ in range(k):
            heads.append(level[0])
            level = np.diff(level, axis=0)
        start = np.stack(heads) if heads else np.zeros((0, inp.shape[1]), dtype=inp.dtype)
        return start, level

    order = np.asarray(order_of_derivative, dtype=np.int64)
    assert order.ndim == 1 and order.shape[0] == inp.shape[1]
    assert (order >= 0).all()
    k_max = int(order.max())
    assert k_max <= inp.shape[0]
    _check_kind(inp, use_decimal)
    n_rows, n_cols = inp.shape[0] - k_max, inp.shape[1]
    start = inp[:k_max].copy()
    diff = _zeros((n_rows, n_cols), use_decimal, inp.dtype if not use_decimal else np.float64)
    for c in range(n_cols):
        col = np.diff(inp[:, c], n=int(order[c]))
        diff[:, c] = col[col.shape[0] - n_rows:]
    return start, diff


def integrate(
    start: np.ndarray, diff: np.ndarray, order_of_derivative: int | np.ndarray, use_decimal: bool
) -> np.ndarray:
    """Inverse of differentiate for either form of `start`."""
    if _is_scalar_order(order_of_derivative):
        k = int(order_of_derivative)
        assert k == start.shape[0]
        _check_kind(start, use_decimal)
        _check_kind(diff, use_decimal)
        out = diff
        for level in range(k - 1, -1, -1):  # innermost difference level first
            out = np.cumsum(np.concatenate((start[level][None], out), axis=0), axis=0)
        return out

    order = np.asarray(order_of_derivative, dtype=np.int64)
    assert order.ndim == 1 and order.shape[0] == diff.shape[1]
    k_max = start.shape[0]
    assert (order <= k_max).all()
    n_rows, n_cols = diff.shape
    out = _zeros((n_rows + k_max, n_cols), use_decimal, diff.dtype if not use_decimal else np.float64)
    for c in range(n_cols):
        k_c = int(order[c])
        raw = start[k_max - k_c:k_max, c] if k_c > 0 else start[:0, c]
        col = diff[:, c]
        for level in range(k_c - 1, -1, -1):
            head = np.diff(raw, n=level)[0]  # first value of the level-th difference
            col = np.cumsum(np.concatenate((np.array([head], dtype=col.dtype), col)))
        if k_max > k_c:  # columns of lower order keep the raw head rows
            col = np.concatenate((start[:k_max - k_c, c], col))
        out[:, c] = col
    return out


# ---------------------------------------------------------------------------
# quantisers (encoder_decoder.py:155-275)
# ---------------------------------------------------------------------------


def _carry_tokens(x: np.ndarray, vocab_size: int, use_decimal: bool) -> np.ndarray:
    """Integer part + difference of the rounded running sum of fractional parts."""
    whole = np.trunc(x)
    acc = np.cumsum(x - whole, axis=0)
    acc = _round_obj(acc) if use_decimal else np.rint(acc)
    carry = np.diff(np.concatenate((np.zeros((1, acc.shape[1]), dtype=acc.dtype), acc), axis=0), axis=0)
    tokens = whole + vocab_size // 2 + carry
    tokens[tokens < 0] = 0
    tokens[tokens >= vocab_size] = vocab_size - 1
    return tokens.astype(np.int64)


def _to_int64(values: np.ndarray, use_decimal: bool) -> np.ndarray:
    if use_decimal:
        return np.array([[int(v) for v in row] for row in values], dtype=np.int64)
    return np.rint(values).astype(np.int64)


def _sigma_delta_k(y: np.ndarray, k: int, vocab_size: int, use_decimal: bool) -> np.ndarray:
    """k-stage MASH cascade of first-order sigma-delta loops.  Stage 0 quantises
    y; stage i quantises minus the error of stage i-1; the stage outputs are
    combined as sum_i (1 - z^-1)^i q_i, so the output minus y is the k-th
    difference of the last stage's error (|e| <= 1/2)."""
    assert k >= 1
    n_rows, n_cols = y.shape
    if use_decimal:
        dtype, zero, rnd = object, Decimal(0), _round_obj
    else:
        dtype, zero, rnd = np.float64, 0.0, np.rint
    q = np.full((k, n_rows, n_cols), zero, dtype=dtype)
    err = np.full((k, n_cols), zero, dtype=dtype)
    for t in range(n_rows):
        feed = y[t]
        for i in range(k):
            target = feed - err[i]
            qi = rnd(target)
            q[i, t] = qi
            e = qi - target
            err[i] = e
            feed = -e
    combined = np.full((n_rows, n_cols), zero, dtype=dtype)
    for i in range(k):
        for j in range(i + 1):
            c = (-1) ** j * math.comb(i, j)
            coef = Decimal(c) if use_decimal else float(c)
            if j == 0:
                combined = combined + coef * q[i]
            else:
                combined[j:] = combined[j:] + coef * q[i, : n_rows - j]
    tokens = _to_int64(combined, use_decimal) + vocab_size // 2
    np.clip(tokens, 0, vocab_size - 1, out=tokens)
    return tokens


def _column_tokens(x: np.ndarray, k: int, vocab_size: int, use_decimal: bool) -> np.ndarray:
    """Per-column quantiser choice; x is (N, 1)."""
    if k == 0:
        r = _round_obj(x) if use_decimal else np.rint(x)
        tokens = _to_int64(r, use_decimal) + vocab_size // 2
        np.clip(tokens, 0, vocab_size - 1, out=tokens)
        return tokens
    if not _uses_cascade(k, vocab_size):
        return _carry_tokens(x, vocab_size, use_decimal)
    return _sigma_delta_k(x, k, vocab_size, use_decimal)


# ---------------------------------------------------------------------------
# public API (encoder_decoder.py:278-427)
# ---------------------------------------------------------------------------


def encode(
    inp: np.ndarray,
    vocab_size: int,
    domain_of_definition: np.ndarray,
    order_of_derivative: int | np.ndarray,
    use_decimal: bool,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(start, scale, tokens): tokens is (T - k_max, F) int64."""
    assert vocab_size % 2 == 0
    assert vocab_size >= 4
    assert domain_of_definition.shape[0] == inp.shape[1]
    n_cols = inp.shape[1]
    _check_kind(inp, use_decimal)
    _check_kind(domain_of_definition, use_decimal)
    if _is_scalar_order(order_of_derivative):
        assert int(order_of_derivative) >= 0
        orders = np.full(n_cols, int(order_of_derivative), dtype=np.int64)
    else:
        orders = np.asarray(order_of_derivative, dtype=np.int64)
        assert orders.shape == (n_cols,)
        assert (orders >= 0).all()

    # scale per column: the domain fills (V - 2)/2 steps, minus 2^k headroom
    # for cascade columns; columns with a zero domain keep scale 1
    scale = np.ones(domain_of_definition.shape, dtype=np.float64)
    if use_decimal:
        scale = np_to_decimal(scale)
    live = np.abs(domain_of_definition) > np.finfo(np.float64).eps
    for c in range(n_cols):
        if not live[c]:
            continue
        k_c = int(orders[c])
        room = vocab_size - 2 - 2**k_c if _uses_cascade(k_c, vocab_size) else vocab_size - 2
        scale[c] = room / domain_of_definition[c] / 2

    start, diff = differentiate(inp, order_of_derivative, use_decimal)
    scaled = diff * scale

    if _is_scalar_order(order_of_derivative):
        k = int(order_of_derivative)
        if _uses_cascade(k, vocab_size):
            return start, scale, _sigma_delta_k(scaled, k, vocab_size, use_decimal)
        return start, scale, _carry_tokens(scaled, vocab_size, use_decimal)

    tokens = np.zeros(scaled.shape, dtype=np.int64)
    for c in range(n_cols):
        tokens[:, c] = _column_tokens(scaled[:, c:c + 1], int(orders[c]), vocab_size, use_decimal)[:, 0]
    return start, scale, tokens


def decode(
    start: np.ndarray,
    scale: np.ndarray,
    inp: np.ndarray,
    vocab_size: int,
    order_of_derivative: int | np.ndarray,
    use_decimal: bool,
) -> np.ndarray:
    """Tokens (N, F) int64 -> series (N + k_max, F)."""
    assert vocab_size % 2 == 0
    assert vocab_size >= 4
    _check_kind(start, use_decimal)
    _check_kind(scale, use_decimal)
    assert inp.dtype == np.int64
    return integrate(start, (inp - vocab_size // 2) / scale, order_of_derivative, use_decimal)


def get_domain_of_definition(
    inp: np.ndarray, order_of_derivative: int | np.ndarray, use_decimal: bool
) -> np.ndarray:
    """Per-column max |k-th difference| (the range the tokens must cover)."""
    _check_kind(inp, use_decimal)
    if _is_scalar_order(order_of_derivative):
        k = int(order_of_derivative)
        assert k >= 0
        return np.max(np.abs(np.diff(inp, n=k, axis=0)), axis=0)
    orders = np.asarray(order_of_derivative, dtype=np.int64)
    assert orders.ndim == 1 and orders.shape[0] == inp.shape[1]
    assert (orders >= 0).all()
    out = _zeros(inp.shape[1], use_decimal)
    for c in range(inp.shape[1]):
        d = np.diff(inp[:, c], n=int(orders[c]))
        if len(d) > 0:
            out[c] = np.max(np.abs(d))
    return out
