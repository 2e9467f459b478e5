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


def test_kv_cache_keys_normed_withdrawn_once_the_tensor_is_exposed():
    # the bounded prefill softmax relies on keys_normed; a caller holding the
    # cache tensor may write arbitrary keys into it at any time, reset included
    c = KVCache(1, 2, 8, 4, 1)
    assert c.keys_normed
    c._tensor()
    assert c.keys_normed  # the library's own accessor leaves it
    c.kv_cache
    assert not c.keys_normed
    c.reset()
    assert not c.keys_normed
    d = KVCache(1, 2, 8, 4, 1)
    d.kv_cache = torch.zeros(1, 2, 1, 2, 8, 4)
    assert not d.keys_normed
    d.reset()
    assert not d.keys_normed
    e = KVCache(1, 2, 8, 4, 1)
    e.keys_normed = False
    e.reset()
    assert e.keys_normed  # the model rewrites every position from 0


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


@pytest.mark.parametrize("n_embd,n_head,ok", [
    (2048, 1, False),  # head_dim 2048: past the largest the kernels take
    (2052, 2, False),  # 1026: even, past 1024
    (1024, 1, True),   # 1024: the largest
    (1024, 2, True),   # 512
    (768, 4, True),    # 192: not a power of two
    (1000, 1, True),   # 1000: not a multiple of a 16-byte slice (pair slices)
    (96, 8, True),     # 12
])
def test_gpt_rejects_head_dims_beyond_the_kernels(n_embd, n_head, ok):
    """The reference's SDPA takes any even head_dim; the HIP kernels take every
    even head_dim up to 1024.  A model outside that range is refused when it
    is built, with the limit in the message, not at its first launch."""
    from diff_gpt import _native

    assert _native.head_dim_supported(n_embd // n_head) == ok
    if ok:
        GPT(vocab_size=64, n_embd=n_embd, block_size=8, n_layer=1, n_head=n_head)
    else:
        with pytest.raises(ValueError, match=r"head_dim \d+ .*even head dims up to 1024"):
            GPT(vocab_size=64, n_embd=n_embd, block_size=8, n_layer=1, n_head=n_head)


def test_projection_weights_are_views_of_one_storage():
    """c_q, c_k, c_v and c_g view one (3*inner + C, C) storage, so no copy of
    them can go stale: updates through .data, in-place ops and load_state_dict
    all land in the GEMM operand, and dtype conversion or a replaced parameter
    re-ties the views."""
    from diff_gpt.model.mha import MultiHeadAttention

    torch.manual_seed(0)
    sa = MultiHeadAttention(n_embd=32, n_head=4, layer_idx=0)
    ws = [sa.c_q.weight, sa.c_k.weight, sa.c_v.weight, sa.c_g.weight]
    fused = sa._projection_weight()
    assert fused.shape == (4 * 32, 32)
    assert all(w.untyped_storage().data_ptr() == fused.untyped_storage().data_ptr() for w in ws)
    assert torch.equal(fused, torch.cat([w.detach() for w in ws]))

    sa.c_k.weight.data.mul_(3.0)  # .data: no _version bump
    with torch.no_grad():
        sa.c_v.weight.add_(1.0)
    assert sa._projection_weight() is fused
    assert torch.equal(fused[32:64], sa.c_k.weight.detach())
    assert torch.equal(fused[64:96], sa.c_v.weight.detach())

    sd = {k: torch.randn_like(v) for k, v in sa.state_dict().items()}
    sa.load_state_dict(sd)
    assert sa._projection_weight() is fused
    assert torch.equal(fused[96:], sd["c_g.weight"]) and torch.equal(fused[:32], sd["c_q.weight"])

    sa = sa.to(torch.bfloat16)
    fused16 = sa._projection_weight()
    assert fused16.dtype == torch.bfloat16
    assert torch.equal(fused16[96:], sd["c_g.weight"].to(torch.bfloat16))
    assert sa.c_q.weight.data_ptr() == fused16.data_ptr()

    new_q = torch.nn.Parameter(torch.ones(32, 32, dtype=torch.bfloat16))
    sa.c_q.weight = new_q
    fused_new = sa._projection_weight()
    assert fused_new is not fused16 and bool((fused_new[:32] == 1).all())
    assert sa.c_q.weight.data_ptr() == fused_new.data_ptr()
    assert list(sa.state_dict()) == ["c_q.weight", "c_k.weight", "c_v.weight", "c_g.weight", "c_proj.weight"]


def test_ordinal_soft_ce_against_float64_loop():
    """The label_smoothing_sigma > 0 loss (gpt.py:15-35): for each kept row,
    -sum_i w_i log softmax(l)_i with w_i proportional to exp(-(i - y)^2 /
    (2 sigma^2)); rows with ignore_index are left out of the mean.  Checked
    against a float64 loop over rows; sigma -> 0 gives the plain
    cross-entropy."""
    import math

    from diff_gpt.model.gpt import _ordinal_soft_ce

    g = torch.Generator().manual_seed(0)
    logits = torch.randn(40, 64, generator=g, dtype=torch.float64) * 3
    targets = torch.randint(0, 64, (40,), generator=g)
    targets[::7] = -100
    for sigma in (0.5, 2.0, 10.0):
        total, n = 0.0, 0
        for row, y in zip(logits.tolist(), targets.tolist()):
            if y == -100:
                continue
            m = max(row)
            lse = m + math.log(sum(math.exp(v - m) for v in row))
            w = [math.exp(-((i - y) ** 2) / (2 * sigma * sigma)) for i in range(64)]
            sw = sum(w)
            total += -sum(wi / sw * (v - lse) for wi, v in zip(w, row))
            n += 1
        got = _ordinal_soft_ce(logits, targets, sigma).item()
        assert abs(got - total / n) <= 1e-12 * max(1.0, abs(total / n))
    keep = targets != -100
    plain = torch.nn.functional.cross_entropy(logits[keep], targets[keep]).item()
    assert abs(_ordinal_soft_ce(logits, targets, 1e-3).item() - plain) <= 1e-9
    assert _ordinal_soft_ce(logits, torch.full((40,), -100), 1.0).item() == 0.0
