"""The forecasting API (diff_gpt.diff_gpt.DiffGPT) on the GPU against the
reference's own outputs (tests/golden/diffgpt.json, written from
fxeqxmulfx/diff-gpt's diff_gpt.py on the CPU with the same seeded cfg0 model
and a greedy sampler): predict (autoregressive and teacher-forced,
diff_gpt.py:127-177, :396-498), predict_samples (:270-293),
predict_quantiles (:365-394) and anomaly_scores (:295-363), plus the
per-column-order Decimal path.  Greedy tokens are integers, so the decoded
forecasts match exactly; anomaly scores are log-probabilities of fp32 logits
and match within 1e-4."""

import json
import math

import numpy as np
import pandas as pd
import pytest
import torch

from conftest import REPO

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((REPO / "tests" / "golden" / "diffgpt.json").read_text())


def _series(seed, rows, cols):
    # the frame of make_golden.py
    rng = np.random.default_rng(seed)
    t = np.arange(rows, dtype=np.float64)[:, None]
    base = np.sin(t * (0.3 + 0.1 * np.arange(cols))) * (1 + np.arange(cols)) + 0.05 * t
    return base + 0.1 * rng.standard_normal((rows, cols))


@pytest.fixture(scope="module")
def setup(dev):
    from diff_gpt import encoder_decoder as ed
    from diff_gpt.diff_gpt import DiffGPT
    from diff_gpt.model.gpt import GPT
    from diff_gpt.sampler.temperature import TemperatureSampler

    kw = json.loads((REPO / "tests" / "golden" / "gpt_weights.json").read_text())["cfg0"]["kwargs"]
    torch.manual_seed(0)
    model = GPT(use_checkpoint=False, **kw).eval().to(dev)
    x = _series(GOLDEN["frame_seed"], GOLDEN["rows"], GOLDEN["cols"])
    df = pd.DataFrame(x, columns=["a", "b", "c"])
    dg = DiffGPT(model, GOLDEN["order"], ed.get_domain_of_definition(x, GOLDEN["order"], False), False)
    return dg, df, x, TemperatureSampler(0.0), model


def test_predict_autoregressive_and_forced(setup):
    dg, df, x, greedy, _ = setup
    got = dg.predict(df, max_new_points=5, sampler=greedy)
    assert list(got.columns) == ["a", "b", "c"] and got.shape == (35, 3)
    assert np.array_equal(got.to_numpy(), np.asarray(GOLDEN["predict"]))
    ctx, fut = df.iloc[:25].reset_index(drop=True), df.iloc[25:].reset_index(drop=True)
    forced = dg.predict(ctx, future_covariates_df=fut, target_columns=["a"], sampler=greedy)
    assert np.array_equal(forced.to_numpy(), np.asarray(GOLDEN["predict_forced"]))


def test_predict_samples_and_quantiles(setup):
    dg, df, _, greedy, _ = setup
    s = dg.predict_samples(df, max_new_points=4, num_samples=3, sampler=greedy)
    assert s.shape == (3, 4, 3)
    assert np.array_equal(s, np.asarray(GOLDEN["samples"]))
    qs = dg.predict_quantiles(df, max_new_points=4, quantiles=(0.1, 0.5, 0.9), num_samples=3,
                              sampler=greedy)
    assert sorted(qs) == [0.1, 0.5, 0.9]
    for q, frame in qs.items():
        assert np.array_equal(frame.to_numpy(), np.asarray(GOLDEN["quantiles"][str(q)]))


def test_anomaly_scores(setup):
    dg, df, _, _, _ = setup
    got = dg.anomaly_scores(df).to_numpy()
    ref = np.asarray([[math.nan if v is None else v for v in row] for row in GOLDEN["anomaly"]])
    assert got.shape == ref.shape
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.abs(got[ok] - ref[ok]).max() <= 1e-4


def test_per_column_orders_decimal(setup):
    from diff_gpt import encoder_decoder as ed
    from diff_gpt.diff_gpt import DiffGPT

    _, df, x, greedy, model = setup
    orders = np.asarray(GOLDEN["percol_decimal_orders"], dtype=np.int64)
    dg = DiffGPT(model, orders, ed.get_domain_of_definition(ed.np_to_decimal(x), orders, True), True)
    got = dg.predict(df, max_new_points=4, sampler=greedy).to_numpy()
    assert np.array_equal(np.asarray(got, dtype=np.float64), np.asarray(GOLDEN["predict_percol_decimal"]))


def test_argument_checks_and_no_training(setup):
    dg, df, _, greedy, _ = setup
    with pytest.raises(AssertionError, match="max_new_points is required"):
        dg.predict(df)
    with pytest.raises(AssertionError, match="block_size"):
        dg.predict(df, max_new_points=100, sampler=greedy)
    with pytest.raises(NotImplementedError):
        dg.train(None)


def test_many_series_in_one_decode_loop(setup):
    """predict_samples_batch and predict_batch decode three series together
    (one prefill, one decode loop, a schedule per series for the forced
    form); greedy, so each series gets exactly what predict_samples /
    predict give it alone -- which the tests above pin to the reference."""
    dg, df, _, greedy, _ = setup
    frames = [df] + [pd.DataFrame(_series(s, GOLDEN["rows"], GOLDEN["cols"]), columns=df.columns) for s in (5, 6)]
    many = dg.predict_samples_batch(frames, max_new_points=4, num_samples=3, sampler=greedy)
    assert many.shape == (3, 3, 4, 3)
    assert np.array_equal(many[0], np.asarray(GOLDEN["samples"]))
    for i, frame in enumerate(frames):
        assert np.array_equal(many[i], dg.predict_samples(frame, max_new_points=4, num_samples=3, sampler=greedy))
    ctxs = [f.iloc[:25].reset_index(drop=True) for f in frames]
    futs = [f.iloc[25:].reset_index(drop=True) for f in frames]
    forced = dg.predict_batch(ctxs, futs, target_columns=["a"], sampler=greedy)
    assert np.array_equal(forced[0].to_numpy(), np.asarray(GOLDEN["predict_forced"]))
    for c, f, got in zip(ctxs, futs, forced):
        one = dg.predict(c, future_covariates_df=f, target_columns=["a"], sampler=greedy)
        assert np.array_equal(got.to_numpy(), one.to_numpy())
