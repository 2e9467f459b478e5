"""The reference's model-level tests, run on the GPU through the HIP path, plus
end-to-end parity with the CPU oracle (oracle.torch_ref).

Ported in spirit from fxeqxmulfx/diff-gpt tests/diff_gpt/model/:
test_rope.py, test_kv_cache.py, test_mha.py, test_block.py, test_gpt.py,
test_engine.py (file:line cited per test).
"""

import math

import numpy as np
import pytest
import torch
from torch.testing import assert_close

from oracle import torch_ref as tr

pytestmark = pytest.mark.gpu


def _fc(seq_len, head_dim, dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    th = torch.randn(1, seq_len, 1, head_dim // 2, generator=g)
    return torch.stack([th.cos(), th.sin()], dim=-1).to(dev)


# ------------------------------------------------------------------ rope (test_rope.py)


def test_rope_pi_over_2(dev):
    from diff_gpt.model.rope import apply_rotary_emb

    x = torch.tensor([[[[1.0, 0.0]]]], device=dev)
    th = torch.tensor([[[[math.pi / 2]]]])
    fc = torch.stack([th.cos(), th.sin()], -1).to(dev)
    assert_close(apply_rotary_emb(x, fc).cpu(), torch.tensor([[[[0.0, 1.0]]]]), atol=1e-6, rtol=1e-6)


def test_rope_explicit_formula(dev):
    # test_rope.py:38-69 with a full (B,H,S,D/2,2) table
    from diff_gpt.model.rope import apply_rotary_emb

    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 4, 8, 16, generator=g)
    th = torch.randn(2, 4, 8, 8, generator=g)
    fc = torch.stack([th.cos(), th.sin()], -1)
    out = apply_rotary_emb(x.to(dev), fc.to(dev)).cpu()
    xr, xi = x[..., 0::2], x[..., 1::2]
    exp = torch.stack([xr * th.cos() - xi * th.sin(), xr * th.sin() + xi * th.cos()], -1).flatten(3)
    assert_close(out, exp)


# ------------------------------------------------------------------ KV cache (test_kv_cache.py)


def test_kv_cache_resize_keeps_contents(dev):
    # test_kv_cache.py:7-81 (head_dim 5, growth on the 5th token)
    from diff_gpt.model.kv_cache import KVCache

    B, H, T, D, L = 2, 3, 4, 5, 6
    c = KVCache(batch_size=B, num_heads=H, seq_len=T, head_dim=D, num_layers=L)

    def put(tok):
        for layer in range(L):
            k = torch.full((B, H, 1, D), float(tok), device=dev)
            c.insert_kv(layer, k, k * 100)

    for i in range(4):
        put(i)
    before = c.kv_cache.clone()
    put(4)
    assert c.kv_cache.shape[4] > before.shape[4]
    for layer in range(L):
        for tok in range(4):
            assert (c.kv_cache[layer, 0, :, :, tok] == tok).all()
            assert (c.kv_cache[layer, 1, :, :, tok] == tok * 100).all()
            assert torch.equal(c.kv_cache[layer, :, :, :, tok], before[layer, :, :, :, tok])


def test_kv_cache_lazy_init_pos_and_chunks(dev):
    # test_kv_cache.py:98-148
    from diff_gpt.model.kv_cache import KVCache

    c = KVCache(1, 2, 10, 8, 2)
    k = torch.randn(1, 2, 1, 8, device=dev)
    c.insert_kv(0, k, k)
    assert c.get_pos() == 0
    k_out, _ = c.insert_kv(1, k, k)
    assert c.get_pos() == 1
    assert_close(k_out[..., 0:1, :], k)
    c2 = KVCache(1, 1, 20, 4, 1)
    kk = torch.randn(1, 1, 5, 4, device=dev)
    out_k, out_v = c2.insert_kv(0, kk, kk * 2)
    assert c2.get_pos() == 5 and out_k.shape[-2] == 5
    assert torch.equal(out_k, kk) and torch.equal(out_v, kk * 2)


def test_kv_cache_growth_rounding(dev):
    # test_kv_cache.py:151-178
    from diff_gpt.model.kv_cache import KVCache

    c = KVCache(1, 1, 10, 4, 1)
    k0 = torch.randn(1, 1, 1, 4, device=dev)
    c.insert_kv(0, k0, k0)
    assert c.kv_cache.shape[4] == 10
    kb = torch.randn(1, 1, 20, 4, device=dev)
    c.insert_kv(0, kb, kb)
    assert c.kv_cache.shape[4] == 2048 and c.get_pos() == 21
    assert torch.equal(c.kv_cache[0, 0, 0, 0, 0], k0[0, 0, 0])
    assert torch.equal(c.kv_cache[0, 0, :, :, 1:21], kb)


def test_kv_cache_prefill_broadcast_and_reset(dev):
    # test_kv_cache.py:181-227
    from diff_gpt.model.kv_cache import KVCache

    src = KVCache(1, 2, 10, 4, 1)
    k = torch.randn(1, 2, 5, 4, device=dev)
    src.insert_kv(0, k, k)
    dst = KVCache(3, 2, 20, 4, 1)
    dst.prefill(src)
    assert dst.get_pos() == 5
    for b in range(3):
        assert torch.equal(dst.kv_cache[0, 0, b, :, :5], k[0])
    src.reset()
    assert src.get_pos() == 0
    one = torch.ones(1, 2, 1, 4, device=dev)
    out_k, _ = src.insert_kv(0, one, one)
    assert torch.equal(out_k, one)


def test_kv_cache_shared_prefix_bookkeeping(dev):
    """A batch-1 -> N prefill records the shared prefix (read once per group by
    decode attention); an insert below it shrinks it, reset() clears it."""
    from diff_gpt.model.kv_cache import KVCache

    src = KVCache(1, 2, 10, 4, 1)
    k = torch.randn(1, 2, 5, 4, device=dev)
    src.insert_kv(0, k, k)
    dst = KVCache(3, 2, 20, 4, 1)
    dst.prefill(src)
    assert dst.shared_prefix == (5, 3)
    step = torch.randn(3, 2, 1, 4, device=dev)
    dst.insert_kv(0, step, step)  # decode step at position 5: prefix untouched
    assert dst.shared_prefix == (5, 3) and dst.get_pos() == 6
    dst.pos = 2  # a rewind (as after a partial reset) makes rows diverge from 2 on
    dst.insert_kv(0, step, step)
    assert dst.shared_prefix == (2, 3)
    dst.reset()
    assert dst.shared_prefix is None
    same = KVCache(1, 2, 20, 4, 1)  # batch 1 -> 1: nothing to share
    same.prefill(src)
    assert same.shared_prefix is None


# ------------------------------------------------------------------ MHA (test_mha.py)


def test_mha_causality(dev):
    # test_mha.py:48-77
    from diff_gpt.model.mha import MultiHeadAttention

    torch.manual_seed(0)
    m = MultiHeadAttention(16, 2, 0).to(dev).eval()
    x = torch.randn(1, 5, 16, device=dev)
    fc = _fc(5, 8, dev)
    with torch.no_grad():
        y0 = m(x, fc, kv_cache=None)
        xp = x.clone()
        xp[:, -1] += 1.0
        y1 = m(xp, fc, kv_cache=None)
    assert_close(y0[:, :-1], y1[:, :-1])
    assert not torch.allclose(y0[:, -1], y1[:, -1])


def test_mha_kv_step_equals_batch(dev):
    # test_mha.py:80-119
    from diff_gpt.model.kv_cache import KVCache
    from diff_gpt.model.mha import MultiHeadAttention

    torch.manual_seed(1)
    m = MultiHeadAttention(16, 2, 0).to(dev).eval()
    x = torch.randn(1, 4, 16, device=dev)
    fc = _fc(4, 8, dev, seed=1)
    kv = KVCache(batch_size=1, num_heads=2, seq_len=10, head_dim=8, num_layers=1)
    with torch.no_grad():
        full = m(x, fc, kv_cache=None)
        steps = [m(x[:, t:t + 1], fc[:, t:t + 1], kv_cache=kv) for t in range(4)]
    assert_close(torch.cat(steps, 1), full, atol=1e-5, rtol=1e-5)


def test_mha_chunked_prefill_then_decode(dev):
    # test_mha.py:122-158, plus a genuine chunk (Tq=3 over Tk=5) that takes the
    # bottom-right mask branch the reference test never reaches
    from diff_gpt.model.kv_cache import KVCache
    from diff_gpt.model.mha import MultiHeadAttention

    torch.manual_seed(2)
    m = MultiHeadAttention(16, 2, 0).to(dev).eval()
    x = torch.randn(1, 6, 16, device=dev)
    fc = _fc(6, 8, dev, seed=2)
    kv = KVCache(batch_size=1, num_heads=2, seq_len=10, head_dim=8, num_layers=1)
    with torch.no_grad():
        full = m(x, fc, None)
        a = m(x[:, :2], fc[:, :2], kv)
        assert kv.get_pos() == 2
        b = m(x[:, 2:5], fc[:, 2:5], kv)
        assert kv.get_pos() == 5
        c = m(x[:, 5:6], fc[:, 5:6], kv)
        assert kv.get_pos() == 6
    assert_close(torch.cat([a, b, c], 1), full, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("D", [64, 128])
def test_mha_bf16_prefill_fused_rope_equals_two_calls(dev, monkeypatch, D):
    """A bf16 prefill with head_dim 64/128 and >= 16 tokens rotates q inside
    the attention launch (dg_prefill_rope), without a cache and with a chunk
    over a KV cache.  With the running-maximum softmax (keys_normed off) the
    output has the bits of the two-call path (the fallback for layouts the
    fused kernel declines); the model's own bounded softmax (every key
    normalised) agrees with it within the bf16 bar."""
    from diff_gpt import _native
    from diff_gpt.model.kv_cache import KVCache
    from diff_gpt.model.mha import MultiHeadAttention

    torch.manual_seed(4)
    H = 2
    m = MultiHeadAttention(H * D, H, 0).to(dev).to(torch.bfloat16).eval()
    x = torch.randn(2, 48, H * D, device=dev).to(torch.bfloat16)
    fc = _fc(48, D, dev, seed=4)
    calls = []
    real = _native.prefill_rope_

    def spy(*a, **k):
        calls.append(1)
        return real(*a, **k)

    def run():
        kv = KVCache(batch_size=2, num_heads=H, seq_len=64, head_dim=D, num_layers=1)
        with torch.no_grad():
            full = m(x, fc, None)
            a = m(x[:, :20], fc[:, :20], kv)
            b = m(x[:, 20:], fc[:, 20:], kv)
        return full, a, b

    monkeypatch.setattr(_native, "prefill_rope_", spy)
    bounded = run()
    assert len(calls) == 3

    def running_max(q, freqs, k, v, y, scale, qknorm, keys_normed=False):
        return real(q, freqs, k, v, y, scale, qknorm, False)

    monkeypatch.setattr(_native, "prefill_rope_", running_max)
    fused = run()
    monkeypatch.setattr(_native, "prefill_rope_", lambda *a, **k: False)
    plain = run()
    for f, b, p in zip(fused, bounded, plain):
        assert torch.equal(f, p)
        assert ((b.float() - p.float()).abs().max() / p.float().abs().max()).item() <= 2e-2


def test_mha_bf16_prefill_over_caller_written_keys(dev, monkeypatch):
    """Keys a caller writes into the cache through its kv_cache tensor carry
    no norm, so the continuation prefill must keep a running maximum: keys 64
    times a normalised row put scores near 2^9 in log2 units, where the
    bounded form's exp2 would overflow.  The result is finite and has the bits
    of the two-call path (rotate q, then the running-maximum kernel)."""
    from diff_gpt import _native
    from diff_gpt.model.kv_cache import KVCache
    from diff_gpt.model.mha import MultiHeadAttention

    torch.manual_seed(5)
    H, D = 2, 64
    m = MultiHeadAttention(H * D, H, 0).to(dev).to(torch.bfloat16).eval()
    x = torch.randn(2, 48, H * D, device=dev).to(torch.bfloat16)
    fc = _fc(48, D, dev, seed=5)
    real = _native.prefill_rope_
    flags = []

    def spy(q, freqs, k, v, y, scale, qknorm, keys_normed=False):
        flags.append(keys_normed)
        return real(q, freqs, k, v, y, scale, qknorm, keys_normed)

    def run():
        kv = KVCache(batch_size=2, num_heads=H, seq_len=64, head_dim=D, num_layers=1)
        with torch.no_grad():
            m(x[:, :20], fc[:, :20], kv)
            kv.kv_cache[0, 0, :, :, :20] *= 64
            return m(x[:, 20:], fc[:, 20:], kv)

    monkeypatch.setattr(_native, "prefill_rope_", spy)
    got = run()
    assert flags == [True, False]
    monkeypatch.setattr(_native, "prefill_rope_", lambda *a, **k: False)
    plain = run()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, plain)


def test_block_kv_step_consistency(dev):
    # test_block.py:129-166 (AttnRes active, layers_per_block=2)
    from diff_gpt.model.block import Block
    from diff_gpt.model.kv_cache import KVCache

    torch.manual_seed(3)
    m = Block(16, 2, 1.0, 10.0, layer_idx=0, layers_per_block=2).to(dev).eval()
    x = torch.randn(1, 6, 16, device=dev)
    fc = _fc(6, 8, dev, seed=3)
    kv = KVCache(batch_size=1, num_heads=2, seq_len=20, head_dim=8, num_layers=1)
    with torch.no_grad():
        _, full = m((x,), x, freqs_cis=fc, kv_cache=None)
        outs = [m((x[:, t:t + 1],), x[:, t:t + 1], freqs_cis=fc[:, t:t + 1], kv_cache=kv)[1]
                for t in range(6)]
    assert_close(torch.cat(outs, 1), full, atol=1e-5, rtol=1e-5)


# ------------------------------------------------------------------ GPT (test_gpt.py)


def _gpt(dev, seed=0, **kw):
    from diff_gpt.model.gpt import GPT

    torch.manual_seed(seed)
    return GPT(**kw).to(dev).eval()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_embd,n_head,lpb", [(64, 4, 1), (128, 4, 2), (512, 8, 1), (512, 8, 3)])
def test_prefill_last_only_equals_full_forward(dev, dtype, n_embd, n_head, lpb):
    """GPT.forward(_last_only=True), the Engine's prefill: the cache holds the
    same bits as after the full forward, and the logits are the full
    forward's last position -- bit for bit where the layers' tails and the
    head are the library's row kernels (n_embd 64, 128), within the
    north-star bars where the tail's GEMMs are hipBLASLt's (a different row
    count may pick another GEMM algorithm)."""
    from diff_gpt.model.kv_cache import KVCache

    model = _gpt(dev, vocab_size=128, n_embd=n_embd, block_size=64, n_head=n_head, n_layer=3,
                 use_checkpoint=False, attn_res_layers_per_block=lpb).to(dtype)
    ids = torch.randint(0, 128, (3, 40), generator=torch.Generator().manual_seed(2)).to(dev)
    D = n_embd // n_head
    kv_full = KVCache(batch_size=3, num_heads=n_head, seq_len=48, head_dim=D, num_layers=3)
    kv_last = KVCache(batch_size=3, num_heads=n_head, seq_len=48, head_dim=D, num_layers=3)
    with torch.no_grad():
        full = model(ids, kv_cache=kv_full)[0][:, -1:]
        last = model.forward(ids, kv_cache=kv_last, _last_only=True)[0]
        nocache = model.forward(ids, _last_only=True)[0]
    assert last.shape == (3, 1, 128)
    assert kv_last.get_pos() == kv_full.get_pos() == 40
    assert torch.equal(kv_last.kv_cache[..., :40, :], kv_full.kv_cache[..., :40, :])
    if n_embd in (64, 128):
        assert torch.equal(last, full)
    else:
        bar = (1e-5 if dtype == torch.float32 else 2e-2) * full.float().abs().max().item()
        assert (last.float() - full.float()).abs().max().item() <= bar
    assert (nocache.float() - last.float()).abs().max().item() <= 2e-2 * last.float().abs().max().item()


def test_gpt_kv_cache_consistency(dev):
    # test_gpt.py:34-76, with two layers and a batch of 3
    from diff_gpt.model.kv_cache import KVCache

    m = _gpt(dev, vocab_size=64, n_embd=16, block_size=20, n_layer=2, n_head=2, use_checkpoint=False)
    idx = torch.randint(0, 64, (3, 5), generator=torch.Generator().manual_seed(0)).to(dev)
    kv = KVCache(batch_size=3, num_heads=2, seq_len=20, head_dim=8, num_layers=2)
    with torch.no_grad():
        full, _ = m(idx)
        steps = [m(idx[:, t:t + 1], kv_cache=kv)[0] for t in range(5)]
    assert_close(full, torch.cat(steps, 1), atol=1e-5, rtol=1e-5)


def test_gpt_generate_length_and_seed(dev):
    # test_gpt.py:102-137
    from diff_gpt.sampler.temperature import TemperatureSampler

    m = _gpt(dev, vocab_size=64, n_embd=32, block_size=16, n_layer=1)
    idx = torch.randint(0, 64, (1, 5), generator=torch.Generator().manual_seed(1)).to(dev)
    assert m.generate(idx, max_new_tokens=3, sampler=None).shape == (1, 8)
    s = TemperatureSampler(temperature=20.0)
    a = m.generate(idx, max_new_tokens=8, sampler=s, seed=7)
    b = m.generate(idx, max_new_tokens=8, sampler=s, seed=7)
    c = m.generate(idx, max_new_tokens=8, sampler=s, seed=99)
    assert torch.equal(a, b) and not torch.equal(a, c)


def test_gpt_softcap_bound(dev):
    # test_gpt.py:188-218
    m = _gpt(dev, vocab_size=64, n_embd=16, block_size=12, n_layer=2, n_head=2)
    with torch.no_grad():
        m.lm_head.weight.mul_(100.0)
        logits, _ = m(torch.randint(0, 64, (2, 6), device=dev))
    assert logits.abs().max().item() <= m.logit_softcap + 1e-5
    assert logits.abs().max().item() >= m.logit_softcap - 1e-3


def test_gpt_rejects_autograd(dev):
    m = _gpt(dev, vocab_size=64, n_embd=16, block_size=12, n_layer=1, n_head=2).train()
    with pytest.raises(RuntimeError, match="inference-only"):
        m(torch.zeros(1, 4, dtype=torch.long, device=dev), torch.zeros(1, 4, dtype=torch.long, device=dev))


# ------------------------------------------------------------------ Engine (test_engine.py)


@pytest.fixture(scope="module")
def engine_model(dev):
    return _gpt(dev, vocab_size=64, n_embd=32, block_size=16, n_head=4, n_layer=2)


def test_engine_shapes_and_determinism(engine_model):
    # test_engine.py:35-121
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    e = Engine(engine_model)
    r, m = e.generate_batch(tokens=[1, 2, 3], num_samples=4, max_tokens=5)
    assert len(r) == 4 and all(len(x) == 8 for x in r) and all(len(x) == 8 for x in m)
    hot = TemperatureSampler(temperature=20)
    r1, _ = e.generate_batch(tokens=[5, 8, 12], num_samples=2, max_tokens=10, seed=42, sampler=hot)
    r2, _ = e.generate_batch(tokens=[5, 8, 12], num_samples=2, max_tokens=10, seed=42, sampler=hot)
    r3, _ = e.generate_batch(tokens=[5, 8, 12], num_samples=2, max_tokens=10, seed=99, sampler=hot)
    assert r1 == r2 and r1 != r3


def test_engine_streaming_equals_batch(engine_model):
    # test_engine.py:124-166
    from diff_gpt.model.engine import Engine

    e = Engine(engine_model)
    rb, mb = e.generate_batch(tokens=[10, 20], num_samples=3, max_tokens=4, seed=123)
    rs = [[10, 20] for _ in range(3)]
    ms = [[0, 0] for _ in range(3)]
    for col, mcol in e.generate(tokens=[10, 20], num_samples=3, max_tokens=4, seed=123):
        for i in range(3):
            rs[i].append(col[i])
            ms[i].append(mcol[i])
    assert rb == rs and mb == ms


def test_engine_ceiling_and_budget(engine_model):
    # test_engine.py:212-247
    from diff_gpt.model.engine import Engine

    e = Engine(engine_model)
    ceil = engine_model.block_size * 2
    r, _ = e.generate_batch(tokens=[1, 2, 3], num_samples=1, max_tokens=ceil - 3 + 50)
    assert len(r[0]) == ceil
    r, _ = e.generate_batch(tokens=[1, 2, 3, 4], num_samples=1)
    assert len(r[0]) == ceil


def test_engine_force_schedule(engine_model):
    # test_engine.py:249-285
    from diff_gpt.model.engine import Engine

    e = Engine(engine_model)
    sched = [7, None, 11, None, 13, None]
    r, m = e.generate_batch(tokens=[1, 2, 3], num_samples=2, max_tokens=6, force_schedule=sched)
    for row, mask in zip(r, m):
        tail = row[3:]
        assert tail[0] == 7 and tail[2] == 11 and tail[4] == 13
        assert mask[3:] == [0, 1, 0, 1, 0, 1]
    r, _ = e.generate_batch(tokens=[1, 2], num_samples=3, max_tokens=4, force_schedule=[5, 6, 7, 8])
    assert all(row[2:] == [5, 6, 7, 8] for row in r)


def test_engine_prefill_clone_equivalence(engine_model):
    # test_engine.py:301-347
    from diff_gpt.model.engine import Engine

    greedy = lambda logits, rng: torch.argmax(logits, dim=-1, keepdim=True)  # noqa: E731
    e = Engine(engine_model)
    many, _ = e.generate_batch(tokens=[1, 8, 4, 9], num_samples=4, max_tokens=6, sampler=greedy)
    one, _ = e.generate_batch(tokens=[1, 8, 4, 9], num_samples=1, max_tokens=6, sampler=greedy)
    assert all(row == many[0] for row in many)
    assert many == one * 4


# ------------------------------------------------------------------ end-to-end parity with the oracle


def _cfg0_model(dev, dtype=torch.float32):
    m = _gpt(dev, vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2,
             use_checkpoint=False)
    return m.to(dtype)


def test_cfg0_greedy_ids_and_logits_match_oracle(dev):
    """fp32, 32 prompts of 96 ids, 48 greedy KV-cache decode
    steps.  Teacher-forced on the oracle's greedy tokens, every step's logits
    agree within 1e-5 * max|ref| (the bar of test_gpt.py:76), and the argmax
    equals the oracle's token for every row whose top-1/top-2 margin exceeds
    twice that bar; rows inside it are near-ties, counted and reported (none
    are expected at these sizes)."""
    from diff_gpt.model.kv_cache import KVCache

    model = _cfg0_model(dev)
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2)
    prompts = torch.randint(0, 256, (32, 96), generator=torch.Generator().manual_seed(1))
    ref_tokens, ref_logits = tr.greedy_decode(params, cfg, prompts, 48)

    kv = KVCache(batch_size=32, num_heads=4, seq_len=144, head_dim=16, num_layers=2)
    worst, near_ties = 0.0, 0
    with torch.no_grad():
        logits, _ = model(prompts.to(dev), kv_cache=kv)
        logits = logits[:, -1]
        for s in range(48):
            ref = ref_logits[s]
            bar = 1e-5 * ref.abs().max().item()
            err = (logits.cpu() - ref).abs().max().item()
            worst = max(worst, err / ref.abs().max().item())
            assert err <= bar, (s, err, bar)
            top2 = ref.topk(2, dim=-1).values
            clear = (top2[:, 0] - top2[:, 1]) > 2 * bar
            near_ties += int((~clear).sum())
            ours = logits.argmax(-1).cpu()
            assert torch.equal(ours[clear], ref_tokens[clear, s])
            logits, _ = model(ref_tokens[:, s:s + 1].to(dev), kv_cache=kv)
            logits = logits[:, -1]
    print(f"cfg0: worst logit error {worst:.3g} x max|ref|, near-ties {near_ties} of {32 * 48}")
    assert near_ties <= 3
    assert kv.get_pos() == 96 + 48


@pytest.mark.parametrize("n_embd,n_head", [(1024, 2), (600, 2), (1024, 1)],
                         ids=["head_dim512", "head_dim300", "head_dim1024"])
def test_wide_head_dim_model_matches_oracle(dev, n_embd, n_head):
    """A GPT whose head_dim is past 256 (the reference's SDPA takes any even
    head_dim; the kernels take every even one up to 1024): fp32 prefill of 3
    prompts of 20 ids and 6 teacher-forced greedy decode steps, logits within
    1e-5 * max|ref| of the oracle at every step and the argmax equal to the
    oracle's token wherever the top-2 margin exceeds twice that bar."""
    from diff_gpt.model.kv_cache import KVCache

    model = _gpt(dev, vocab_size=64, n_embd=n_embd, block_size=40, n_head=n_head, n_layer=1,
                 use_checkpoint=False)
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=64, n_embd=n_embd, block_size=40, n_head=n_head, n_layer=1)
    prompts = torch.randint(0, 64, (3, 20), generator=torch.Generator().manual_seed(5))
    ref_tokens, ref_logits = tr.greedy_decode(params, cfg, prompts, 6)
    kv = KVCache(batch_size=3, num_heads=n_head, seq_len=26, head_dim=n_embd // n_head, num_layers=1)
    with torch.no_grad():
        logits = model(prompts.to(dev), kv_cache=kv)[0][:, -1]
        for s in range(6):
            ref = ref_logits[s]
            bar = 1e-5 * ref.abs().max().item()
            err = (logits.cpu() - ref).abs().max().item()
            assert err <= bar, (s, err, bar)
            top2 = ref.topk(2, dim=-1).values
            clear = (top2[:, 0] - top2[:, 1]) > 2 * bar
            assert torch.equal(logits.argmax(-1).cpu()[clear], ref_tokens[clear, s])
            logits = model(ref_tokens[:, s:s + 1].to(dev), kv_cache=kv)[0][:, -1]


def test_cfg0_kv_cache_contents_match_oracle(dev):
    """After the cfg0 prefill, the cache holds the oracle's rotated+normed K and
    raw V (same model weights; the projections differ only by GEMM rounding)."""
    from diff_gpt.model.kv_cache import KVCache

    model = _cfg0_model(dev)
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2)
    prompts = torch.randint(0, 256, (8, 96), generator=torch.Generator().manual_seed(2))
    kv = KVCache(batch_size=8, num_heads=4, seq_len=96, head_dim=16, num_layers=2)
    with torch.no_grad():
        model(prompts.to(dev), kv_cache=kv)
        ref = tr.RefCache(8, 4, 96, 16, 2)
        tr.forward(params, cfg, prompts, ref)
    assert_close(kv.kv_cache.cpu(), ref.data, atol=2e-5, rtol=1e-4)


def test_bf16_model_logits_close_to_oracle(dev):
    """cfg0/1 model cast to bf16 (freqs table included, gpt.py buffer .to()):
    prefill + 8 teacher-forced decode steps.  bf16 rounding through two layers
    moves softcapped logits by a few tenths whatever the device, so the bar is
    relative to that noise: against the same bf16 weights evaluated in fp32
    (the exact model), the HIP path may deviate at most 1.5x as much as the
    reference's own bf16 CPU evaluation does, and stays within 2e-2 of the
    largest exact logit."""
    from diff_gpt.model.kv_cache import KVCache

    model = _cfg0_model(dev, torch.bfloat16)
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    params32 = {k: v.float() for k, v in params.items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2)
    prompts = torch.randint(0, 256, (16, 96), generator=torch.Generator().manual_seed(3))
    _, bf_logits = tr.greedy_decode(params, cfg, prompts, 8)
    tokens = torch.stack([l.argmax(-1) for l in bf_logits], 1)
    _, exact = tr.greedy_decode(params32, cfg, prompts, 8, forced=tokens.T.tolist())
    kv = KVCache(batch_size=16, num_heads=4, seq_len=104, head_dim=16, num_layers=2)
    worst_ours, worst_ref = 0.0, 0.0
    with torch.no_grad():
        logits = model(prompts.to(dev), kv_cache=kv)[0][:, -1]
        for s in range(8):
            worst_ours = max(worst_ours, (logits.float().cpu() - exact[s]).abs().max().item())
            worst_ref = max(worst_ref, (bf_logits[s].float() - exact[s]).abs().max().item())
            logits = model(tokens[:, s:s + 1].to(dev), kv_cache=kv)[0][:, -1]
    span = max(e.abs().max().item() for e in exact)
    print(f"bf16 cfg0 model: worst |logit err| ours {worst_ours:.4g}, reference bf16 {worst_ref:.4g}, "
          f"max|exact| {span:.4g}")
    assert worst_ours <= 1.5 * worst_ref + 1e-3, (worst_ours, worst_ref)
    assert worst_ours <= 2e-2 * span, (worst_ours, span)


# ------------------------------------------------------------------ captured decode step


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_step_kernels_match_plain(dev, dtype):
    """dg_rope_qknorm_append_at / dg_decode_attention_at (position read on the
    device) write and compute exactly what the plain kernels do at that
    position, and write nothing for a position past the cache."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, D, cap, pos = 6, 4, 16, 40, 23
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(B, 1, H, D, generator=g).to(dtype).to(dev) for _ in range(3))
    table = precompute_freqs_cis(D, 2 * cap, 10000).to(dtype).to(dev)
    base = torch.randn(2, B, H, cap, D, generator=g).to(dtype).to(dev)
    c1, c2 = base.clone(), base.clone()
    ops = _native.ops()
    # plain: explicit window at pos
    q1 = torch.empty_like(q)
    ops.rope_qknorm_append(q, k, v, table[pos:pos + 1].view(1, 1, 1, D // 2, 2), q1,
                           c1[0, :, :, pos:pos + 1].transpose(1, 2), c1[1, :, :, pos:pos + 1].transpose(1, 2), True)
    y1 = ops.attention(q1, c1[0, :, :, :pos + 1].transpose(1, 2), c1[1, :, :, :pos + 1].transpose(1, 2), D ** -0.5)
    # device position
    p = torch.tensor([pos], dtype=torch.int32, device=dev)
    q2, y2 = torch.empty_like(q), torch.empty_like(q)
    _native.rope_qknorm_append_at_(q, k, v, table, q2, c2[0].transpose(1, 2), c2[1].transpose(1, 2), p, True)
    _native.decode_attention_at_(q2, c2[0].transpose(1, 2), c2[1].transpose(1, 2), y2, D ** -0.5, p)
    assert torch.equal(q1, q2) and torch.equal(c1, c2) and torch.equal(y1, y2)
    # out-of-range position: nothing written
    c3 = base.clone()
    _native.rope_qknorm_append_at_(q, k, v, table, q2, c3[0].transpose(1, 2), c3[1].transpose(1, 2),
                                   torch.tensor([cap], dtype=torch.int32, device=dev), True)
    torch.cuda.synchronize()
    assert torch.equal(c3, base)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_engine_graph_replay_equals_eager(dev, dtype):
    """The captured decode step replayed once per step (with the sampler, the
    H2D token copy and host syncs between replays) reproduces the eager
    engine token for token: greedy, forced steps, and temperature-1 sampling
    with the same seed (identical logits -> identical draws)."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.model.gpt import GPT
    from diff_gpt.sampler.temperature import TemperatureSampler

    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2,
                use_checkpoint=False).eval().to(dev).to(dtype)
    prompt = torch.randint(0, 256, (40,), generator=torch.Generator().manual_seed(3)).tolist()
    schedule = [None, 5, None, None, 9, None, None, None]
    for kw in (dict(sampler=TemperatureSampler(0.0)),
               dict(sampler=TemperatureSampler(0.0), force_schedule=schedule),
               dict(sampler=TemperatureSampler(1.0), seed=7)):
        a = Engine(model).generate_batch(prompt, num_samples=12, max_tokens=8, **kw)
        b = Engine(model, use_graph=False).generate_batch(prompt, num_samples=12, max_tokens=8, **kw)
        assert a == b, kw


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_engine_kept_graph_equals_eager_across_calls(dev, dtype):
    """One Engine over several generate_multi_batch calls with the same rows,
    prompt length and budget (the captured step kept and replayed again):
    other seeds and temperatures, forced and per-row mixed steps between
    sampled ones -- tokens and masks equal to the eager engine's every time."""
    import numpy as np

    from diff_gpt.model.engine import Engine
    from diff_gpt.model.gpt import GPT
    from diff_gpt.sampler.temperature import TemperatureSampler

    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2,
                use_checkpoint=False).eval().to(dev).to(dtype)
    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, 256, (30,), generator=g).tolist() for _ in range(3)]
    rows, steps = 3 * 8, 12
    table = np.random.default_rng(5).integers(0, 256, (rows, steps))
    table[np.random.default_rng(6).random((rows, steps)) < 0.6] = -1  # sampled where negative
    table[:, 3] = 17  # every row forced
    cases = [dict(sampler=TemperatureSampler(1.0), seed=1),
             dict(sampler=TemperatureSampler(1.0), seed=2),
             dict(sampler=TemperatureSampler(0.7), seed=3),
             dict(sampler=None, seed=4),
             dict(sampler=TemperatureSampler(0.0)),
             dict(sampler=TemperatureSampler(1.0), seed=5, force_schedule=[None, 5, None, None, 9] + [None] * 7),
             dict(sampler=TemperatureSampler(1.3), seed=6, force_schedule=table)]
    e = Engine(model)
    kept = None
    for kw in cases:
        got = e.generate_multi_batch(prompts, num_samples=8, max_tokens=steps, **kw)
        ref = Engine(model, use_graph=False).generate_multi_batch(prompts, num_samples=8, max_tokens=steps, **kw)
        assert got == ref, kw
        assert kept is None or e._kept[2] is kept  # one capture, replayed by every later call
        kept = e._kept[2]


def test_engine_reuses_the_captured_step_across_calls(dev):
    """A second call with the same rows, prompt length and budget replays the
    step captured by the first into the same cache, and gives a fresh Engine's
    tokens; a different prompt length or an in-place weight change captures
    anew."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.sampler.temperature import TemperatureSampler

    model = _gpt(dev, vocab_size=64, n_embd=32, block_size=32, n_head=4, n_layer=2)
    hot = TemperatureSampler(temperature=3.0)
    prompts = ([5, 8, 12, 1], [7, 7, 2, 30], [9, 1])
    e = Engine(model)
    for seed, p in zip((1, 2, 3), prompts):
        got, _ = e.generate_batch(tokens=p, num_samples=24, max_tokens=9, seed=seed, sampler=hot)
        ref, _ = Engine(model).generate_batch(tokens=p, num_samples=24, max_tokens=9, seed=seed, sampler=hot)
        assert got == ref
    graph = e._kept[2]
    e.generate_batch(tokens=[9, 3], num_samples=24, max_tokens=9, seed=4, sampler=hot)
    assert e._kept[2] is graph  # same key: the captured step was replayed
    e.generate_batch(tokens=[9, 3, 4], num_samples=24, max_tokens=9, seed=4, sampler=hot)
    assert e._kept[2] is not graph  # another prompt length: captured anew
    graph = e._kept[2]
    with torch.no_grad():
        model.blocks[1].sa.c_v.weight.mul_(-1.5)
    got, _ = e.generate_batch(tokens=[9, 3, 4], num_samples=24, max_tokens=9, seed=5, sampler=hot)
    assert e._kept[2] is not graph  # parameters changed in place: captured anew
    ref, _ = Engine(model).generate_batch(tokens=[9, 3, 4], num_samples=24, max_tokens=9, seed=5, sampler=hot)
    assert got == ref
