"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

Each oracle function is checked against something independent of its own
formula: the reference's known-answer tests, torch library routines on the CPU
(the very calls the reference makes), float64 closed forms, or invariants.
The reference ships no golden files; its test modules hold the known answers
reused here (paths relative to fxeqxmulfx/diff-gpt/tests/diff_gpt/model/).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import numerics as on
from oracle import torch_ref as tr


def _ulp_diff_f32(a: np.ndarray, b: np.ndarray) -> int:
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return int(np.abs(ai - bi).max()) if ai.size else 0


# ---------------------------------------------------------------- rounding


def test_bf16_round_matches_torch_and_known_bits():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.4e38, 1e-40], np.float32),
    ])
    ours = on.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    # ties go to even: 1 + 2^-8 lies halfway between bf16 1.0 and 1 + 2^-7
    assert on.bf16_round(np.array([1.0 + 2**-8], np.float32))[0] == 1.0
    assert on.bf16_round(np.array([1.0 + 3 * 2**-8], np.float32))[0] == 1.0 + 2**-6
    assert np.isnan(on.bf16_round(np.array([np.nan], np.float32))[0])


# ---------------------------------------------------------------- RoPE table


def test_freqs_table_known_answers():
    # test_rope_freqs.py:21-53
    t = on.freqs_table_f64(4, 2, 10000)
    assert t.shape == (2, 2, 2)
    assert np.allclose(t[0, :, 0], 1.0) and np.allclose(t[0, :, 1], 0.0)
    assert math.isclose(t[1, 0, 0], math.cos(1.0)) and math.isclose(t[1, 0, 1], math.sin(1.0))
    assert math.isclose(t[1, 1, 0], math.cos(0.01)) and math.isclose(t[1, 1, 1], math.sin(0.01))
    big = on.freqs_table_f64(20, 10, 10000)
    assert np.allclose(np.hypot(big[..., 0], big[..., 1]), 1.0)


@pytest.mark.parametrize("dim,end", [(16, 276), (64, 4096), (128, 4096)])
def test_host_freqs_table_close_to_exact(dim, end):
    """The product builds the table with torch on the host (gpt.py:131-135);
    it sits within a few fp32 ulps of the exact table (angles up to ~4e3 rad
    amplify the fp32 rounding of m*w_j, hence an absolute bound)."""
    from diff_gpt.model.rope import precompute_freqs_cis

    ours = precompute_freqs_cis(dim, end, 10000).numpy().astype(np.float64)
    exact = on.freqs_table_f64(dim, end, 10000)
    ang = np.arange(end)[:, None] * (1.0 / 10000 ** (np.arange(0, dim, 2) / dim))[None]
    tol = 4 * np.finfo(np.float32).eps * np.maximum(1.0, ang)[..., None]
    assert np.all(np.abs(ours - exact) <= tol)
    # and it is the very table the oracle's torch restatement builds
    assert torch.equal(precompute_freqs_cis(dim, end, 10000), tr.freqs_table(dim, end, 10000))


# ---------------------------------------------------------------- RoPE


def test_rope_pi_over_2_known_answer():
    # test_rope.py:14-35: (1, 0) rotated by pi/2 is (0, 1)
    cs = np.array([[math.cos(math.pi / 2), math.sin(math.pi / 2)]], np.float32)
    out = on.rope(np.array([1.0, 0.0], np.float32), cs, "f32")
    assert abs(out[0]) < 1e-6 and abs(out[1] - 1.0) < 1e-6


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rope_equals_reference_torch_ops_bitwise(dtype):
    """The reference's own ops (rope.py:20-27) on the CPU give the same bits:
    mul, mul, sub/add are each rounded in both."""
    g = torch.Generator().manual_seed(1)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    x = torch.randn(3, 7, 4, 16, generator=g).to(tdt)
    theta = torch.randn(1, 7, 1, 8, generator=g)
    fc = torch.stack([theta.cos(), theta.sin()], dim=-1).to(tdt)
    ref = tr.rope(x, fc).float().numpy()
    ours = on.rope(x.float().numpy(), fc.float().numpy(), dtype)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_rope_close_to_fp64_rotation():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 32)).astype(np.float32)
    th = rng.standard_normal((5, 16))
    cs = np.stack([np.cos(th), np.sin(th)], -1).astype(np.float32)
    out = on.rope(x, cs, "f32").astype(np.float64)
    xr, xi = x[:, 0::2].astype(np.float64), x[:, 1::2].astype(np.float64)
    c, s = cs[..., 0].astype(np.float64), cs[..., 1].astype(np.float64)
    exact = np.stack([xr * c - xi * s, xr * s + xi * c], -1).reshape(5, 32)
    assert np.abs(out - exact).max() < 4e-7 * np.abs(x).max()


# ---------------------------------------------------------------- RMSNorm


def test_tree_sum_order():
    v = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    # ((1e8 + 1) + (-1e8 + 1)) in fp32: both pairs round away the 1s
    assert on.tree_sum(v) == np.float32(0.0)
    assert on.tree_sum(np.arange(5, dtype=np.float32)) == 10.0


@pytest.mark.parametrize("n", [5, 8, 16, 64, 128, 1024])
def test_rms_norm_f32_against_torch(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(257, n, generator=g) * 3
    ref = F.rms_norm(x, (n,)).numpy()
    ours = on.rms_norm(x.numpy(), "f32")
    # torch's (unspecified) reduction order and ours differ by a few ulps
    assert _ulp_diff_f32(ours, ref) <= 4
    # closed form in fp64 with eps = FLT_EPSILON (not the 1e-6 the reference's
    # test_rms_norm.py:17 comment assumes): both stay within 3 ulps of it
    xd = x.double().numpy()
    exact = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + np.finfo(np.float32).eps)
    ulps = np.abs(ours - exact) / np.spacing(np.abs(exact).astype(np.float32))
    assert ulps.max() <= 3.0


def test_rms_norm_bf16_against_torch():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4096, 64, generator=g).to(torch.bfloat16)
    ref = F.rms_norm(x, (64,)).float().numpy()
    ours = on.rms_norm(x.float().numpy(), "bf16")
    # one fp32 ulp of difference before rounding can flip a bf16 tie
    diff = np.abs(ours - ref)
    assert (diff <= np.abs(ref) * 2**-8 + 1e-30).all()
    assert (diff == 0).mean() > 0.99


def test_rms_norm_invariants():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((10, 100)) * 10).astype(np.float32)
    y = on.rms_norm(x, "f32")
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, atol=1e-3)
    assert np.allclose(on.rms_norm(5 * x, "f32"), y, atol=1e-5, rtol=1e-4)


# ---------------------------------------------------------------- float64 models


@pytest.mark.parametrize("table", [torch.float64, torch.float32])
def test_rope_f64_matches_torch_type_promotion(table):
    """rope.py:20-27 on float64 rows, run by torch on the CPU: x.float() then
    the table's promotion (float64 table: float64 products; fp32 table: fp32
    products, widened by type_as).  Bit for bit for both table dtypes, and the
    two differ, so a mistaken promotion fails one of them."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, 9, 4, 24, generator=g, dtype=torch.float64) * 3
    theta = torch.randn(1, 9, 1, 12, generator=g, dtype=torch.float64) * 4
    fc = torch.stack([theta.cos(), theta.sin()], dim=-1).to(table)
    ref = tr.rope(x, fc).numpy()
    assert tr.rope(x, fc).dtype == torch.float64
    ours = on.rope_f64(x.numpy(), fc.numpy())
    assert np.array_equal(ours.view(np.uint64), ref.view(np.uint64))
    other = on.rope_f64(x.numpy(), fc.numpy().astype(np.float32 if table == torch.float64 else np.float64))
    assert not np.array_equal(other, ours)


def test_rope_f64_rounds_input_to_fp32_and_quarter_turn():
    # x.float(): 1 + 2^-40 is 1.0 in fp32, so angle 0 returns exactly 1.0
    out = on.rope_f64(np.array([1.0 + 2**-40, 0.0]), np.array([[1.0, 0.0]]))
    assert out[0] == 1.0 and out[1] == 0.0
    # test_rope.py:14-35: (1, 0) by pi/2 -> (cos, sin) of pi/2 in float64
    out = on.rope_f64(np.array([1.0, 0.0]), np.array([[math.cos(math.pi / 2), math.sin(math.pi / 2)]]))
    assert abs(out[0]) < 1e-16 and out[1] == 1.0


@pytest.mark.parametrize("n", [6, 64, 1000])
def test_rms_norm_f64_against_torch(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(129, n, generator=g, dtype=torch.float64) * 5
    ref = F.rms_norm(x, (n,)).numpy()
    ours = on.rms_norm_f64(x.numpy())
    assert np.abs(ours - ref).max() <= 8 * np.finfo(np.float64).eps * np.abs(ref).max()
    assert np.allclose(np.sqrt((ours ** 2).mean(-1)), 1.0, rtol=0, atol=1e-14)


# ---------------------------------------------------------------- attention


@pytest.mark.parametrize("Tq,Tk", [(9, 9), (1, 13), (4, 11)])
def test_attention_f64_matches_torch_sdpa(Tq, Tk):
    g = torch.Generator().manual_seed(Tq * 100 + Tk)
    B, H, D = 2, 3, 8
    q = torch.randn(B, H, Tq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, Tk, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, Tk, D, generator=g, dtype=torch.float64)
    ref = tr.sdpa(q, k, v).transpose(1, 2).numpy()
    ours = on.attention_f64(
        q.transpose(1, 2).numpy(), k.transpose(1, 2).numpy(), v.transpose(1, 2).numpy()
    )
    assert np.abs(ours - ref).max() < 1e-12


def test_attention_f64_closed_forms():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 1, 1, 4))
    k = np.repeat(rng.standard_normal((1, 1, 1, 4)), 6, axis=1)  # identical keys
    v = rng.standard_normal((1, 6, 1, 4))
    out = on.attention_f64(q, k, v)  # uniform weights
    assert np.allclose(out[0, 0, 0], v[0, :, 0].mean(0))
    # causal row 0 sees only key 0
    q2 = rng.standard_normal((1, 3, 1, 4))
    k2 = rng.standard_normal((1, 3, 1, 4))
    v2 = rng.standard_normal((1, 3, 1, 4))
    assert np.allclose(on.attention_f64(q2, k2, v2)[0, 0], v2[0, 0])


@pytest.mark.parametrize("Tq,Tk", [(40, 40), (1, 37), (13, 50)])
def test_attention_head_f64_equals_brute_force(Tq, Tk):
    """The per-head matrix-product form against attention_f64 (causal, decode
    and chunked masks), whole and restricted to a slice of the queries."""
    rng = np.random.default_rng(Tq + 7 * Tk)
    D = 16
    q, k, v = rng.standard_normal((Tq, D)), rng.standard_normal((Tk, D)), rng.standard_normal((Tk, D))
    ref = on.attention_f64(q[None, :, None], k[None, :, None], v[None, :, None])[0, :, 0]
    assert np.abs(on.attention_head_f64(q, k, v) - ref).max() < 1e-12
    sl = slice(Tq // 2, Tq)
    assert np.abs(on.attention_head_f64(q, k, v, rows=sl) - ref[sl]).max() < 1e-12


# ---------------------------------------------------------------- KV cache model


def test_cache_model_known_answers():
    # test_kv_cache.py:7-81 (fill values survive growth), :151-178 (21 -> 2048)
    c = on.CacheModel(B=2, H=3, T=4, D=5, L=6)
    for tok in range(5):
        for layer in range(6):
            kk = np.full((2, 3, 1, 5), float(tok), np.float32)
            c.insert(layer, kk, kk * 100)
    assert c.pos == 5 and c.data.shape[4] == on.grown_capacity(5) == 2048
    for tok in range(5):
        assert (c.data[:, 0, :, :, tok] == tok).all()
        assert (c.data[:, 1, :, :, tok] == 100 * tok).all()
    assert on.grown_capacity(21) == 2048
    # pos advances only after the last layer (test_kv_cache.py:98-126)
    c2 = on.CacheModel(1, 2, 10, 8, 2)
    c2.insert(0, np.zeros((1, 2, 1, 8), np.float32), np.zeros((1, 2, 1, 8), np.float32))
    assert c2.pos == 0
    c2.insert(1, np.zeros((1, 2, 1, 8), np.float32), np.zeros((1, 2, 1, 8), np.float32))
    assert c2.pos == 1
    # prefill broadcast 1 -> 3 (test_kv_cache.py:181-204)
    src = on.CacheModel(1, 2, 10, 4, 1)
    kk = np.random.default_rng(6).standard_normal((1, 2, 5, 4)).astype(np.float32)
    src.insert(0, kk, kk)
    dst = on.CacheModel(3, 2, 20, 4, 1)
    dst.prefill(src)
    assert dst.pos == 5
    for b in range(3):
        assert np.array_equal(dst.data[0, 0, b, :, :5], kk[0])


# ---------------------------------------------------------------- model restatement


def _tiny_params(cfg: tr.ModelConfig, seed=0):
    from diff_gpt.model.gpt import GPT

    torch.manual_seed(seed)
    m = GPT(vocab_size=cfg.vocab_size, n_embd=cfg.n_embd, block_size=cfg.block_size,
            n_head=cfg.n_head, n_layer=cfg.n_layer, use_checkpoint=False,
            attn_res_layers_per_block=cfg.attn_res_layers_per_block)
    return {k: v.detach() for k, v in m.state_dict().items()}


@pytest.mark.parametrize("lpb", [1, 2])
def test_torch_ref_kv_decode_equals_full_forward(lpb):
    """test_gpt.py:34-76's invariant holds for the restated model."""
    cfg = tr.ModelConfig(vocab_size=64, n_embd=32, block_size=20, n_head=4, n_layer=3,
                         attn_res_layers_per_block=lpb)
    p = _tiny_params(cfg)
    idx = torch.randint(0, 64, (2, 7), generator=torch.Generator().manual_seed(7))
    with torch.no_grad():
        full = tr.forward(p, cfg, idx)
        cache = tr.RefCache(2, 4, 20, 8, 3)
        steps = [tr.forward(p, cfg, idx[:, t:t + 1], cache) for t in range(7)]
        chunk_cache = tr.RefCache(2, 4, 20, 8, 3)
        c1 = tr.forward(p, cfg, idx[:, :3], chunk_cache)
        c2 = tr.forward(p, cfg, idx[:, 3:], chunk_cache)  # chunked branch, Tq=4 < Tk=7
    torch.testing.assert_close(torch.cat(steps, 1), full, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(torch.cat([c1, c2], 1), full, atol=1e-5, rtol=1e-5)
