"""Engine.generate_multi / generate_multi_batch: several prompts of one length
decoded together (one batched prefill, each prompt's cache stored once and
shared by its rows, one captured decode step for all rows), with force
schedules shared, per prompt or per row.

The reference decodes one prompt per call with one schedule for all rows
(engine.py:87, :108-124).  These tests pin the multi-prompt loop to that
path: with a greedy sampler every row's tokens must equal the single-prompt
Engine's for its own prompt and its own schedule (identical logits per row,
so identical argmax), and a per-row schedule whose rows all carry the
reference's schedule must give the reference's own output
(tests/golden/engine_greedy.json, written from fxeqxmulfx/diff-gpt).  The
models are fp32: the projections run as GEMMs over all rows, and a different
row count may round the logits differently in their last bits; in fp32 that
cannot move an argmax away from a clear maximum."""

import json

import numpy as np
import pytest
import torch

from conftest import REPO

pytestmark = pytest.mark.gpu


def _model(dev, dtype=torch.float32, **kw):
    from diff_gpt.model.gpt import GPT

    cfg = dict(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2)
    cfg.update(kw)
    torch.manual_seed(0)
    return GPT(use_checkpoint=False, **cfg).eval().to(dev).to(dtype)


def _prompts(n, length, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 256, (length,), generator=g).tolist() for _ in range(n)]


@pytest.mark.parametrize("num_samples", [1, 5, 20])
@pytest.mark.parametrize("use_graph", [True, False], ids=["graph", "eager"])
def test_multi_greedy_equals_per_prompt_calls(dev, num_samples, use_graph):
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    model = _model(dev)
    prompts = _prompts(3, 20, 1)
    greedy = TemperatureSampler(0.0)
    res, masks = Engine(model, use_graph=use_graph).generate_multi_batch(
        prompts, num_samples=num_samples, max_tokens=12, sampler=greedy)
    assert len(res) == 3 * num_samples
    for p, prompt in enumerate(prompts):
        one, one_masks = Engine(model).generate_batch(prompt, num_samples=num_samples, max_tokens=12, sampler=greedy)
        assert res[p * num_samples:(p + 1) * num_samples] == one
        assert masks[p * num_samples:(p + 1) * num_samples] == one_masks


def test_multi_per_prompt_schedules(dev):
    """Each prompt with a schedule of its own (configs[4]'s pattern: a few
    channel positions forced per step): every prompt's rows equal the
    single-prompt Engine with that schedule, masks 0 at forced steps."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    model = _model(dev)
    prompts = _prompts(4, 21, 2)
    steps = 14
    rng = np.random.default_rng(3)
    schedules = [[int(rng.integers(0, 256)) if (21 + s + p) % 7 in (0, 1, 2) else None for s in range(steps)]
                 for p in range(4)]
    greedy = TemperatureSampler(0.0)
    res, masks = Engine(model).generate_multi_batch(prompts, num_samples=3, max_tokens=steps, sampler=greedy,
                                                    force_schedule=schedules)
    for p, prompt in enumerate(prompts):
        one, one_masks = Engine(model).generate_batch(prompt, num_samples=3, max_tokens=steps, sampler=greedy,
                                                      force_schedule=schedules[p])
        assert res[3 * p:3 * p + 3] == one
        assert masks[3 * p:3 * p + 3] == one_masks
        for s, tok in enumerate(schedules[p]):
            if tok is not None:
                assert all(r[21 + s] == tok and m[21 + s] == 0 for r, m in zip(res[3 * p:3 * p + 3],
                                                                               masks[3 * p:3 * p + 3]))


def test_per_row_schedule_with_equal_rows_is_the_reference_output(dev):
    """A per-row schedule table whose rows all carry the reference's shared
    schedule reproduces the reference's own results and masks; so does the
    per-prompt list form and the shared list form of generate_multi."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler
    from test_gpu_golden import _model as golden_model

    doc = json.loads((REPO / "tests" / "golden" / "engine_greedy.json").read_text())
    model, _ = golden_model(doc["model"], dev)
    f = doc["forced"]
    n = f["num_samples"]
    row = [-1 if t is None else t for t in f["force_schedule"]]
    table = np.array([row] * n, dtype=np.int64)
    greedy = TemperatureSampler(0.0)
    e = Engine(model)
    for sched in (table, [f["force_schedule"]], f["force_schedule"]):
        res, masks = e.generate_multi_batch([doc["prompt"]], num_samples=n, max_tokens=f["max_tokens"],
                                            sampler=greedy, force_schedule=sched)
        assert res == f["results"] and masks == f["masks"]


def test_mixed_per_row_schedule(dev):
    """Rows of one prompt with different forced positions: a step where some
    rows are forced keeps their scheduled token (mask 0) and takes the
    sampled one elsewhere (mask 1).  Greedy, so each row equals a
    single-row Engine call with that row's schedule."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    model = _model(dev)
    prompts = _prompts(2, 16, 4)
    steps, N = 10, 4
    rng = np.random.default_rng(5)
    table = np.where(rng.random((2 * N, steps)) < 0.35, rng.integers(0, 256, (2 * N, steps)), -1)
    table[:, 0] = 9        # a step forcing every row
    table[:, 1] = -1       # a step sampling every row
    greedy = TemperatureSampler(0.0)
    res, masks = Engine(model).generate_multi_batch(prompts, num_samples=N, max_tokens=steps, sampler=greedy,
                                                    force_schedule=table)
    for r in range(2 * N):
        sched = [None if t < 0 else int(t) for t in table[r]]
        one, one_masks = Engine(model).generate_batch(prompts[r // N], num_samples=1, max_tokens=steps,
                                                      sampler=greedy, force_schedule=sched)
        assert res[r] == one[0], r
        assert masks[r] == one_masks[0], r
        assert masks[r][16:] == [0 if t >= 0 else 1 for t in table[r]]


def test_multi_sampling_is_seeded_and_streams(dev):
    """Temperature-1 sampling over 4 prompts x 25 rows: the same seed gives
    the same tokens (a kept captured step is reused by the second call), the
    streaming form yields the same columns, another seed differs."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    model = _model(dev)
    prompts = _prompts(4, 30, 6)
    hot = TemperatureSampler(1.0)
    e = Engine(model)
    a = e.generate_multi_batch(prompts, num_samples=25, max_tokens=9, sampler=hot, seed=3)
    kept = e._kept[2]
    b = e.generate_multi_batch(prompts, num_samples=25, max_tokens=9, sampler=hot, seed=3)
    assert e._kept[2] is kept and a == b
    cols = [c for c, _ in e.generate_multi(prompts, num_samples=25, max_tokens=9, sampler=hot, seed=3)]
    assert [row[30:] for row in a[0]] == [list(x) for x in zip(*cols)]
    c = e.generate_multi_batch(prompts, num_samples=25, max_tokens=9, sampler=hot, seed=4)
    assert c[0] != a[0]
    assert all(len(r) == 39 for r in a[0]) and all(m == [0] * 30 + [1] * 9 for m in a[1])


def test_multi_argument_checks(dev):
    from diff_gpt.model.engine import Engine

    model = _model(dev)
    e = Engine(model)
    with pytest.raises(AssertionError, match="same length"):
        e.generate_multi_batch([[1, 2, 3], [4, 5]], num_samples=2, max_tokens=3)
    with pytest.raises(AssertionError, match="one schedule per prompt"):
        e.generate_multi_batch([[1, 2], [4, 5]], num_samples=2, max_tokens=3, force_schedule=[[1, 2, 3]])
    with pytest.raises(AssertionError, match="cover all generation steps"):
        e.generate_multi_batch([[1, 2], [4, 5]], num_samples=2, max_tokens=3, force_schedule=[[1], [2]])
    with pytest.raises(AssertionError, match="per-row force_schedule"):
        e.generate_multi_batch([[1, 2], [4, 5]], num_samples=2, max_tokens=3,
                               force_schedule=np.zeros((3, 3), dtype=np.int64))
