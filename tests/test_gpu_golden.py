"""The product path on the GPU against the reference's own outputs
(tests/golden/, written from fxeqxmulfx/diff-gpt on the CPU):

  * GPT.forward logits without and with a KV cache: fp32 within
    1e-5 x max|ref| (gpt.py:140-200);
  * the KV-cache greedy decode of test_gpt.py:34-76: identical token ids
    (each step's top-1/top-2 margin is checked first so that a tie could not
    make the comparison meaningless), per-step logits within 1e-5, and the
    cache contents within 1e-5 x max|ref|;
  * Engine.generate_batch with a greedy sampler, with and without
    force_schedule (engine.py:29-169): identical ids and masks.
"""

import json

import numpy as np
import pytest
import torch

from conftest import REPO

pytestmark = pytest.mark.gpu

GOLDEN = REPO / "tests" / "golden"
CASES = [("cfg0", (2, 8), 4), ("lpb2", (2, 7), 3)]


def _model(name, dev):
    from diff_gpt.model.gpt import GPT

    kw = json.loads((GOLDEN / "gpt_weights.json").read_text())[name]["kwargs"]
    torch.manual_seed(0)
    return GPT(use_checkpoint=False, **kw).eval().to(dev), kw


def _rel(a, ref):
    return float(np.abs(np.asarray(a, np.float64) - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("name,shape,steps", CASES)
def test_gpt_matches_reference_outputs(dev, name, shape, steps):
    from diff_gpt.model.kv_cache import KVCache

    z = np.load(GOLDEN / "gpt_forward.npz")
    model, kw = _model(name, dev)
    B, T = shape
    H, D, L = kw["n_head"], kw["n_embd"] // kw["n_head"], kw["n_layer"]
    ids = torch.from_numpy(z[f"{name}_ids"]).to(dev)
    with torch.no_grad():
        full, _ = model(ids)
        assert _rel(full.cpu().numpy(), z[f"{name}_full_logits"]) <= 1e-5
        pre, _ = model(ids, kv_cache=KVCache(B, H, T, D, L))
        assert _rel(pre.cpu().numpy(), z[f"{name}_prefill_logits"]) <= 1e-5

        cache = KVCache(batch_size=B, num_heads=H, seq_len=T + steps, head_dim=D, num_layers=L)
        logits, _ = model(ids, kv_cache=cache)
        last = logits[:, -1]
        ref_steps = z[f"{name}_step_logits"]
        ref_toks = z[f"{name}_greedy_tokens"]
        for s in range(steps):
            assert _rel(last.cpu().numpy(), ref_steps[:, s]) <= 1e-5
            top2 = torch.topk(torch.from_numpy(ref_steps[:, s]), 2, dim=-1).values
            assert ((top2[:, 0] - top2[:, 1]) > 1e-4).all(), "near-tie: ids not comparable"
            nxt = last.argmax(dim=-1)
            assert nxt.cpu().numpy().tolist() == ref_toks[:, s].tolist()
            logits, _ = model(nxt[:, None], kv_cache=cache)
            last = logits[:, -1]
        assert _rel(last.cpu().numpy(), ref_steps[:, steps]) <= 1e-5
    assert cache.get_pos() == int(z[f"{name}_cache_pos"])
    got = cache.kv_cache.cpu().numpy()
    assert got.shape == z[f"{name}_cache"].shape
    assert _rel(got, z[f"{name}_cache"]) <= 1e-5


def test_engine_matches_reference_greedy_and_forced(dev):
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    doc = json.loads((GOLDEN / "engine_greedy.json").read_text())
    model, _ = _model(doc["model"], dev)
    engine = Engine(model)
    f = doc["forced"]
    res, masks = engine.generate_batch(doc["prompt"], num_samples=f["num_samples"],
                                       max_tokens=f["max_tokens"], sampler=TemperatureSampler(0.0),
                                       force_schedule=f["force_schedule"])
    assert res == f["results"] and masks == f["masks"]
    fr = doc["free"]
    res, masks = engine.generate_batch(doc["prompt"], num_samples=fr["num_samples"],
                                       max_tokens=fr["max_tokens"], sampler=TemperatureSampler(0.0))
    assert res == fr["results"] and masks == fr["masks"]
