"""Host-side behaviour of the drop-in package that needs no GPU: argument
validation with the reference's assertion messages, the RoPE-ceiling budget,
KVCache bookkeeping, state_dict compatibility, and the absence of any CPU
fallback on the attention path."""

import pytest
import torch

from diff_gpt.model.engine import Engine
from diff_gpt.model.gpt import GPT
from diff_gpt.model.kv_cache import KVCache, _grown_capacity
from diff_gpt.model.rms_norm import rms_norm
from diff_gpt.model.rope import apply_rotary_emb, precompute_freqs_cis


@pytest.fixture(scope="module")
def cpu_model():
    m = GPT(vocab_size=64, n_embd=32, block_size=16, n_head=4, n_layer=2)
    return m.eval()


# engine.py:51-53 messages, as matched by test_engine.py:173-188
def test_engine_rejects_empty_prompt(cpu_model):
    with pytest.raises(AssertionError, match="non-empty"):
        Engine(cpu_model).generate_batch(tokens=[], num_samples=1, max_tokens=2)


def test_engine_rejects_mixed_type_tokens(cpu_model):
    with pytest.raises(AssertionError, match="list of ints"):
        Engine(cpu_model).generate_batch(tokens=[1, 2, 3.0], num_samples=1, max_tokens=2)


def test_engine_force_schedule_too_short(cpu_model):
    with pytest.raises(AssertionError, match="force_schedule must cover"):
        Engine(cpu_model).generate_batch(
            tokens=[1, 2, 3], num_samples=1, max_tokens=10, force_schedule=[1, 2, 3]
        )


def test_engine_early_return_at_rope_ceiling(cpu_model):
    # test_engine.py:191-209: no prefill, no allocation, rows are the prompt
    prompt = list(range(cpu_model.block_size * 2))
    results, masks = Engine(cpu_model).generate_batch(tokens=prompt, num_samples=2, max_tokens=10)
    assert results == [prompt, prompt] and masks == [[0] * len(prompt)] * 2


def test_engine_budget_clamps(cpu_model):
    e = Engine(cpu_model)
    assert e._budget(3, 4) == 4
    assert e._budget(3, 10_000) == 2 * 16 - 3
    assert e._budget(4, None) == 2 * 16 - 4


def test_kv_cache_initial_state():
    # test_kv_cache.py:84-95
    c = KVCache(2, 4, 128, 64, 3)
    assert c.get_pos() == 0 and c.kv_cache.size(0) == 0
    assert c.kv_shape == (3, 2, 2, 4, 128, 64)
    c.pos = 7
    c.reset()
    assert c.get_pos() == 0


def test_kv_cache_prefill_assertions():
    a, b = KVCache(3, 2, 20, 4, 1), KVCache(1, 2, 10, 4, 1)
    with pytest.raises(AssertionError, match="Cannot prefill with a None KV cache"):
        a.prefill(b)
    b.kv_cache = torch.zeros(1, 2, 1, 2, 10, 4)
    a.kv_cache = torch.zeros(1)
    with pytest.raises(AssertionError, match="Cannot prefill a non-empty KV cache"):
        a.prefill(b)
    c = KVCache(3, 5, 20, 4, 1)
    with pytest.raises(AssertionError, match="Head count mismatch"):
        c.prefill(b)
    d = KVCache(3, 2, 5, 4, 1)
    with pytest.raises(AssertionError, match="Sequence length mismatch"):
        d.prefill(b)


def test_growth_rule():
    # kv_cache.py:92-96; test_kv_cache.py:151-178
    assert _grown_capacity(21) == 2048
    assert _grown_capacity(5) == 2048
    assert _grown_capacity(1024) == 2048
    assert _grown_capacity(1025) == 3072


def test_no_cpu_fallback_on_the_hot_path():
    x = torch.randn(1, 4, 2, 8)
    fc = precompute_freqs_cis(8, 4, 10000).view(1, 4, 1, 4, 2)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        apply_rotary_emb(x, fc)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        rms_norm(x)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        KVCache(1, 2, 4, 8, 1).insert_kv(0, x.transpose(1, 2), x.transpose(1, 2))
    m = GPT(vocab_size=64, n_embd=16, block_size=8, n_layer=1, n_head=2).eval()
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm devices only"):
        m(torch.zeros(1, 3, dtype=torch.long))


def test_state_dict_keys_match_reference_layout():
    """Module names/order of gpt.py:117-135, block.py:58-72, mha.py:25-29,
    feed_forward.py:10-14: reference checkpoints load unchanged."""
    m = GPT(vocab_size=64, n_embd=16, block_size=8, n_layer=2, n_head=2)
    expected = ["token_embedding_table.weight"]
    for i in range(2):
        expected += [f"blocks.{i}.sa.c_{n}.weight" for n in ("q", "k", "v", "g", "proj")]
        expected += [f"blocks.{i}.ffwd.net.0.weight", f"blocks.{i}.ffwd.net.2.weight",
                     f"blocks.{i}.attn_res_proj.weight", f"blocks.{i}.mlp_res_proj.weight"]
    expected += ["lm_head.weight"]
    assert list(m.state_dict().keys()) == expected
    assert m.lm_head.weight is m.token_embedding_table.weight
    assert "freqs_cis" not in m.state_dict()


def test_gpt_constructor_assertions():
    with pytest.raises(AssertionError, match="multiple of"):
        GPT(vocab_size=70, n_embd=16, block_size=8, n_layer=1, n_head=2)
    GPT(vocab_size=70, n_embd=16, block_size=8, n_layer=1, n_head=2, pad_vocab_size_to=1)
    with pytest.raises(AssertionError, match="label_smoothing_sigma"):
        GPT(vocab_size=64, n_embd=16, n_layer=1, n_head=2, label_smoothing_sigma=-0.1)
