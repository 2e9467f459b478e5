"""Samplers (src/diff_gpt/sampler/{temperature,nucleus}.py) on host and device
logits.

The properties are those of the reference's own tests
(tests/diff_gpt/sampler/test_nucleus_sampler.py:7-132,
test_temperature_sampler.py:50-63): the (B, 1) shape, determinism under a
seeded generator, sampled tokens confined to the nucleus, p = 1 equal to the
inner sampler, p -> 0 equal to argmax.  The kept set itself is pinned against
an independent numpy construction of the nucleus (sort descending, keep a
rank while the mass before it is below p), read back through a recording
inner sampler.  Each test runs on the CPU and, marked ``gpu``, on the ROCm
device with a device generator, which is where the Engine calls the samplers.
"""

import numpy as np
import pytest
import torch

from diff_gpt.sampler.nucleus import NucleusSampler
from diff_gpt.sampler.temperature import TemperatureSampler

DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]


def _gen(device, seed):
    return torch.Generator(device=device).manual_seed(seed)


def _randn(shape, seed, device):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(device)


class _Recorder:
    """Inner sampler that keeps the logits it was handed and returns argmax."""

    def __init__(self):
        self.seen = None

    def __call__(self, logits, rng=None):
        self.seen = logits.clone()
        return torch.argmax(logits, dim=-1, keepdim=True)


def _nucleus_np(logits: np.ndarray, p: float) -> np.ndarray:
    """Boolean keep-mask of the nucleus, built row by row in float64."""
    keep = np.zeros(logits.shape, dtype=bool)
    for r, row in enumerate(logits.astype(np.float64)):
        e = np.exp(row - row.max())
        prob = e / e.sum()
        order = np.argsort(-prob, kind="stable")
        mass = 0.0
        for rank, idx in enumerate(order):
            if rank > 0 and not mass < p:
                break
            keep[r, idx] = True
            mass += prob[idx]
    return keep


@pytest.mark.parametrize("device", DEVICES)
def test_output_shape(device):
    logits = _randn((4, 50), 0, device)
    out = NucleusSampler(0.9, TemperatureSampler(1.0))(logits, rng=_gen(device, 0))
    assert out.shape == (4, 1) and out.dtype == torch.int64 and out.device.type == device


@pytest.mark.parametrize("device", DEVICES)
def test_determinism_with_rng(device):
    logits = _randn((2, 100), 1, device)
    s = NucleusSampler(0.9, TemperatureSampler(1.5))
    a = s(logits, rng=_gen(device, 42))
    b = s(logits, rng=_gen(device, 42))
    assert torch.equal(a, b)
    # a different seed gives a different draw for some row over a few tries
    differs = any(not torch.equal(a, s(logits, rng=_gen(device, seed))) for seed in (99, 100, 101))
    assert differs


@pytest.mark.parametrize("device", DEVICES)
def test_nucleus_selection_logic(device):
    """P = [0.6, 0.25, 0.1, 0.05], p = 0.9: the nucleus is {0, 1, 2}; every
    sample is in it and, over 2000 draws, each of its tokens appears."""
    probs = torch.tensor([[0.6, 0.25, 0.1, 0.05]])
    logits = torch.log(probs).to(device).expand(2000, -1)
    s = NucleusSampler(0.9, TemperatureSampler(1.0))
    got = set(torch.unique(s(logits, rng=_gen(device, 123))).tolist())
    assert got == {0, 1, 2}


@pytest.mark.parametrize("device", DEVICES)
def test_p_equals_one_is_inner_sampler(device):
    logits = _randn((10, 20), 2, device)
    inner = TemperatureSampler(1.2)
    a = inner(logits, rng=_gen(device, 1337))
    b = NucleusSampler(1.0, inner)(logits, rng=_gen(device, 1337))
    assert torch.equal(a, b)


@pytest.mark.parametrize("device", DEVICES)
def test_p_tiny_is_argmax(device):
    logits = _randn((4, 30), 3, device)
    got = NucleusSampler(1e-9, TemperatureSampler(2.0))(logits, rng=_gen(device, 5))
    assert torch.equal(got, torch.argmax(logits, dim=-1, keepdim=True))


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("p", [0.3, 0.9, 0.99])
def test_kept_set_matches_numpy_nucleus(device, p):
    """The logits handed to the inner sampler keep exactly the nucleus of an
    independent float64 construction (rows of the model's vocabulary size,
    with a few peaked rows) and are -inf elsewhere."""
    logits = _randn((64, 256), 4, device) * 2.0
    logits[:8] *= 6.0  # peaked rows: nuclei of one or two tokens
    rec = _Recorder()
    NucleusSampler(p, rec)(logits)
    seen = rec.seen.cpu().numpy()
    expect = _nucleus_np(logits.cpu().numpy(), p)
    kept = np.isfinite(seen)
    # float32 cumulative sums can flip the one rank whose mass sits within
    # rounding of p; no such rank exists in these rows
    assert np.array_equal(kept, expect)
    assert np.array_equal(seen[kept], logits.cpu().numpy()[kept])


@pytest.mark.parametrize("device", DEVICES)
def test_temperature_zero_is_first_argmax(device):
    """T = 0 takes the first maximum (temperature.py:22-23), ties included."""
    logits = _randn((6, 256), 6, device)
    logits[:, 7] = 50.0
    logits[:, 200] = 50.0
    got = TemperatureSampler(0.0)(logits)
    assert got.shape == (6, 1) and bool((got == 7).all())


@pytest.mark.gpu
def test_predict_samples_with_nucleus(dev):
    """DiffGPT.predict_samples with the README's sampling setting (top-p 0.9
    over temperature 1): seeded runs repeat exactly, the shape is
    (num_samples, new points, columns), the values are finite, and the draws
    differ between trajectories."""
    import json

    import pandas as pd

    from conftest import REPO
    from diff_gpt import encoder_decoder as ed
    from diff_gpt.diff_gpt import DiffGPT
    from diff_gpt.model.gpt import GPT

    kw = json.loads((REPO / "tests" / "golden" / "gpt_weights.json").read_text())["cfg0"]["kwargs"]
    torch.manual_seed(0)
    model = GPT(use_checkpoint=False, **kw).eval().to(dev)
    rng = np.random.default_rng(3)
    t = np.arange(30, dtype=np.float64)[:, None]
    x = np.sin(t * np.array([0.3, 0.5])) + 0.1 * rng.standard_normal((30, 2))
    df = pd.DataFrame(x, columns=["a", "b"])
    dg = DiffGPT(model, 1, ed.get_domain_of_definition(x, 1, False), False)
    sampler = NucleusSampler(0.9, TemperatureSampler(1.0))
    a = dg.predict_samples(df, max_new_points=6, num_samples=16, sampler=sampler)
    b = dg.predict_samples(df, max_new_points=6, num_samples=16, sampler=sampler)
    assert a.shape == (16, 6, 2)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b)
    assert len({tuple(row) for row in a.reshape(16, -1)}) > 1


def _gen_state(g):
    return g.get_state()


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(6400, 256), (7, 50), (256,), (3, 1)])
def test_draw_one_equals_torch_multinomial(device, dtype, shape):
    """draw_one reproduces torch.multinomial(probs, 1, generator) bit for bit --
    the same ids and the generator left in the same state -- on softmax
    probabilities, on rows with zero entries (as the nucleus leaves them),
    one-hot rows, and a 1-D distribution; with a generator and with the
    default one."""
    from diff_gpt.sampler.temperature import draw_one

    logits = _randn(shape, 31 + len(shape), device).to(dtype)
    probs = torch.softmax(logits, dim=-1)
    if len(shape) == 2 and shape[1] > 2:
        probs[: shape[0] // 2, ::3] = 0  # zero entries
        probs[-1] = 0
        probs[-1, -1] = 1  # one-hot row
    for seed in (0, 5, 123):
        g1, g2 = _gen(device, seed), _gen(device, seed)
        want = torch.multinomial(probs, num_samples=1, generator=g1)
        got = draw_one(probs, g2)
        assert got.shape == want.shape and got.dtype == want.dtype
        assert torch.equal(got, want), seed
        assert torch.equal(_gen_state(g1), _gen_state(g2))
        # again from the state both generators are left in
        assert torch.equal(draw_one(probs, g2), torch.multinomial(probs, num_samples=1, generator=g1))
    torch.manual_seed(9)
    want = torch.multinomial(probs, num_samples=1)
    torch.manual_seed(9)
    assert torch.equal(draw_one(probs), want)


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("temperature", [1.0, 0.7, 3.0])
def test_temperature_sampler_equals_reference_formula(device, temperature):
    """TemperatureSampler(T) returns the reference's
    torch.multinomial(softmax(logits / T), 1, generator) ids, T = 1 included
    (where it skips the division: x / 1 is x)."""
    logits = _randn((500, 256), 77, device)
    for dtype in (torch.float32, torch.bfloat16):
        x = logits.to(dtype)
        want = torch.multinomial(torch.softmax(x / temperature, dim=-1), num_samples=1, generator=_gen(device, 4))
        got = TemperatureSampler(temperature)(x, rng=_gen(device, 4))
        assert torch.equal(got, want)
