"""The sigma-delta tokenizer (diff_gpt.encoder_decoder) against the
reference's own outputs (tests/golden/codec.json, written from
fxeqxmulfx/diff-gpt's encoder_decoder.py:278-427): tokens, start rows, scales,
domains and decoded series are identical, bit for bit in float64 and digit
for digit in Decimal, for shared and per-column orders and every quantiser
(plain rounding, carry, MASH cascade).  Independent of the golden data:
decode(encode(x)) stays within the quantiser's error bound (the invariant of
the reference's tests/diff_gpt/test_encoder_decoder.py round trips)."""

import json
from decimal import Decimal

import numpy as np
import pytest

from conftest import REPO

GOLDEN = json.loads((REPO / "tests" / "golden" / "codec.json").read_text())


def _dec(obj):
    shape = tuple(obj["shape"])
    if "decimal" in obj:
        flat = obj["decimal"]
        vals = [Decimal(v) for row in flat for v in (row if isinstance(row, list) else [row])]
        out = np.empty(len(vals), dtype=object)
        out[:] = vals
        return out.reshape(shape)
    if "int" in obj:
        return np.asarray(obj["int"], dtype=np.int64).reshape(shape)
    return np.asarray([float(v) for v in obj["float"]], dtype=np.float64).reshape(shape)


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape
    if a.dtype == object or b.dtype == object:
        assert [str(x) for x in a.reshape(-1)] == [str(x) for x in b.reshape(-1)]
    else:
        assert a.dtype == b.dtype
        assert np.array_equal(a.view(np.int64) if a.dtype == np.float64 else a,
                              b.view(np.int64) if b.dtype == np.float64 else b)


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_codec_matches_reference(name):
    from diff_gpt import encoder_decoder as ed

    case = GOLDEN[name]
    x = _dec(case["input"])
    dec = case["use_decimal"]
    order = np.asarray(case["order"], dtype=np.int64) if isinstance(case["order"], list) else case["order"]
    xin = ed.np_to_decimal(x) if dec else x
    domain = ed.get_domain_of_definition(xin, order, dec)
    _same(domain, _dec(case["domain"]))
    start, scale, tokens = ed.encode(xin, case["vocab"], domain, order, dec)
    _same(start, _dec(case["start"]))
    _same(scale, _dec(case["scale"]))
    _same(tokens, _dec(case["tokens"]))
    assert tokens.min() >= 0 and tokens.max() < case["vocab"]
    back = ed.decode(start, scale, tokens, case["vocab"], order, dec)
    _same(back, _dec(case["decoded"]))


@pytest.mark.parametrize("k", [0, 1, 2, 3])
def test_round_trip_error_bound(k):
    """MASH (k >= 2): decoded - x = (k-th integral of (k-th difference of an
    error bounded by 1/2)) / scale, i.e. bounded by 2^(k-1)/scale; k <= 1:
    the carry scheme keeps the cumulative rounding error below 1/scale."""
    from diff_gpt import encoder_decoder as ed

    rng = np.random.default_rng(100 + k)
    x = np.cumsum(rng.standard_normal((400, 2)), axis=0)
    vocab = 256
    domain = ed.get_domain_of_definition(x, k, False)
    start, scale, tokens = ed.encode(x, vocab, domain, k, False)
    back = ed.decode(start, scale, tokens, vocab, k, False)
    assert back.shape == x.shape
    bound = (2.0 ** max(k - 1, 0) + 1e-6) / scale
    assert (np.abs(back - x) <= bound[None, :] + 1e-9 * np.abs(x).max()).all()


def test_integrate_inverts_differentiate_per_column():
    from diff_gpt import encoder_decoder as ed

    rng = np.random.default_rng(7)
    x = rng.standard_normal((15, 3))
    order = np.asarray([2, 0, 3], dtype=np.int64)
    start, diff = ed.differentiate(x, order, False)
    assert start.shape == (3, 3) and diff.shape == (12, 3)
    assert np.allclose(ed.integrate(start, diff, order, False), x, atol=1e-12)
    xd = ed.np_to_decimal(x)
    sd, dd = ed.differentiate(xd, order, True)
    back = ed.integrate(sd, dd, order, True)
    # Decimal's 28-digit context rounds the long binary expansions of the floats
    err = max(abs(back[i, j] - xd[i, j]) for i in range(15) for j in range(3))
    assert err < Decimal("1e-24")
