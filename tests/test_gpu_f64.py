"""float64 models (GPT.double()) on the GPU through the C-ABI.

The reference's SDPA, rms_norm and rotary embedding take float64 tensors
(mha.py:61-81, rms_norm.py:5-7, rope.py:20-27); the library runs them on
float64 vector-ALU kernels.  Bars:
  * the rotation alone: bit for bit against oracle.numerics.rope_f64, for a
    float64 table (float64 products) and an fp32 table (fp32 products);
  * the QK-norm and the row kernels: within 16 float64 ulps of max|ref| of the
    oracle (their reduction order is the kernel's, not numpy's);
  * attention: within 1e-12 * max|ref| of float64 brute force (a few thousand
    rounded float64 terms per output);
  * the model: logits within 1e-10 * max|ref| of the oracle's float64 forward
    (hipBLASLt / rocBLAS float64 GEMMs in their own summation order), greedy
    ids equal wherever the top-2 margin exceeds twice that bar.
"""

import numpy as np
import pytest
import torch

from oracle import numerics as on
from oracle import torch_ref as tr

pytestmark = pytest.mark.gpu

EPS = np.finfo(np.float64).eps
ATTN_TOL = 1e-12
MODEL_TOL = 1e-10


def _randn(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64) * scale


def _rel(got: torch.Tensor, ref: np.ndarray) -> float:
    return float(np.abs(got.cpu().numpy() - ref).max() / np.abs(ref).max())


# ------------------------------------------------------------------ RoPE + QK-norm + append


@pytest.mark.parametrize("table", ["f64", "f32"])
@pytest.mark.parametrize("D", [8, 12, 64, 128, 300, 1024])
def test_rope_qknorm_append_f64(dev, table, D):
    """Rotated q and k bit for bit (qknorm off) or within 16 ulps (qknorm on)
    of the oracle; v copied exactly into the cache page at pos; the rest of the
    cache untouched."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, T, H, pos, cap = 3, 7, 2, 5, 16
    q, k, v = (_randn((B, T, H, D), 40 + D + i, 3.0) for i in range(3))
    fdt = torch.float64 if table == "f64" else torch.float32
    fc = precompute_freqs_cis(D, 64, 10000).to(fdt)[pos:pos + T].view(1, T, 1, D // 2, 2)
    fcn = np.broadcast_to(fc.numpy(), (B, T, H, D // 2, 2))
    exp_q, exp_k = on.rope_f64(q.numpy(), fcn), on.rope_f64(k.numpy(), fcn)
    ops = _native.ops()
    for qknorm in (False, True):
        cache = torch.full((2, B, H, cap, D), 7.0, dtype=torch.float64, device=dev)
        q_out = torch.empty((B, T, H, D), dtype=torch.float64, device=dev)
        k_dst = cache[0, :, :, pos:pos + T].transpose(1, 2)
        v_dst = cache[1, :, :, pos:pos + T].transpose(1, 2)
        ops.rope_qknorm_append(q.to(dev), k.to(dev), v.to(dev), fc.to(dev), q_out, k_dst, v_dst, qknorm)
        got_k = cache[0, :, :, pos:pos + T].transpose(1, 2).cpu().numpy()
        if qknorm:
            for got, exp in ((q_out.cpu().numpy(), on.rms_norm_f64(exp_q)), (got_k, on.rms_norm_f64(exp_k))):
                assert np.abs(got - exp).max() <= 16 * EPS * np.abs(exp).max()
        else:
            assert np.array_equal(q_out.cpu().numpy().view(np.uint64), exp_q.view(np.uint64))
            assert np.array_equal(got_k.view(np.uint64), exp_k.view(np.uint64))
        assert torch.equal(cache[1, :, :, pos:pos + T].transpose(1, 2).cpu(), v)
        rest = cache.cpu().clone()
        rest[:, :, :, pos:pos + T] = 7.0
        assert (rest == 7.0).all()


def test_rope_only_f64_broadcast_table(dev):
    """apply_rotary_emb (the product module) on float64 rows with a float64
    table that broadcasts over batch and heads: bit for bit."""
    from diff_gpt.model.rope import apply_rotary_emb

    x = _randn((2, 4, 8, 10), 3)
    th = _randn((1, 1, 8, 5), 4)
    fc = torch.stack([th.cos(), th.sin()], -1)
    out = apply_rotary_emb(x.to(dev), fc.to(dev))
    exp = on.rope_f64(x.numpy(), np.broadcast_to(fc.numpy(), (2, 4, 8, 5, 2)))
    assert out.dtype == torch.float64
    assert np.array_equal(out.cpu().numpy().view(np.uint64), exp.view(np.uint64))


@pytest.mark.parametrize("N", [5, 64, 1000, 8192])
def test_rms_norm_f64(dev, N):
    from diff_gpt.model.rms_norm import rms_norm

    x = _randn((5, 9, N), N, 4.0)
    y = rms_norm(x.to(dev))
    exp = on.rms_norm_f64(x.numpy())
    assert y.dtype == torch.float64
    assert np.abs(y.cpu().numpy() - exp).max() <= 16 * EPS * np.abs(exp).max()


# ------------------------------------------------------------------ attention

ATTN = [  # (B, H, Tq, Tk, D)
    (2, 3, 1, 700, 64),     # decode
    (4, 2, 1, 3000, 128),   # long decode
    (2, 2, 96, 96, 16),     # causal prefill
    (1, 2, 200, 330, 64),   # chunked prefill (prefix + lower triangle)
    (1, 1, 1, 1, 8),        # one key
    (2, 1, 40, 40, 1000),   # wide head
    (1, 2, 1, 500, 300),
]


@pytest.mark.parametrize("shape", ATTN, ids=lambda s: "x".join(map(str, s)))
def test_attention_f64(dev, shape):
    """dg_attention in float64 against float64 brute force (all three mask
    branches), with k and v as strided views of a cache page."""
    from diff_gpt import _native

    B, H, Tq, Tk, D = shape
    q = _randn((B, Tq, H, D), Tq + D)
    cache = _randn((2, B, H, Tk + 9, D), Tk + D, 2.0)
    keys, vals = cache[0, :, :, :Tk].transpose(1, 2), cache[1, :, :, :Tk].transpose(1, 2)
    ref = on.attention_f64(q.numpy(), keys.numpy(), vals.numpy())
    cd = cache.to(dev)
    y = _native.ops().attention(q.to(dev), cd[0, :, :, :Tk].transpose(1, 2), cd[1, :, :, :Tk].transpose(1, 2),
                                1.0 / np.sqrt(D))
    assert y.dtype == torch.float64
    err = _rel(y, ref)
    assert err <= ATTN_TOL, err


def test_attention_f64_scale_is_carried_as_fp32(dev):
    """The ABI carries the scale as fp32: SDPA's default 1/sqrt(D) stands for
    itself in float64, any other scale acts as its fp32 rounding."""
    from diff_gpt import _native

    B, H, Tq, Tk, D = 2, 2, 1, 300, 128
    q, k, v = _randn((B, Tq, H, D), 1, 3.0), _randn((B, Tk, H, D), 2, 3.0), _randn((B, Tk, H, D), 3)
    ops = _native.ops()
    y = ops.attention(q.to(dev), k.to(dev), v.to(dev), 1.0 / np.sqrt(D))
    assert _rel(y, on.attention_f64(q.numpy(), k.numpy(), v.numpy())) <= ATTN_TOL
    y = ops.attention(q.to(dev), k.to(dev), v.to(dev), 0.3)
    ref = on.attention_f64(q.numpy(), k.numpy(), v.numpy(), scale=float(np.float32(0.3)))
    assert _rel(y, ref) <= ATTN_TOL


@pytest.mark.parametrize("shape", [(7, 3, 2, 40, 90, 64), (5, 5, 1, 16, 17, 16)], ids=lambda s: "x".join(map(str, s)))
def test_attention_f64_shared_prefix(dev, shape):
    """A prefix shared by groups of rows (dg_prefix) gives the bits of the
    rows holding it themselves, and float64 attention within the bar."""
    from diff_gpt import _native

    B, G, H, P, Tk, D = shape
    groups = (B + G - 1) // G
    cache = _randn((2, B, H, Tk, D), 5 + D)
    cache[:, :, :, :P] = _randn((groups, 2, H, P, D), 6 + D).repeat_interleave(G, dim=0)[:B].transpose(0, 1)
    q = _randn((B, 1, H, D), 7 + D, 2.0)
    cd, qd = cache.to(dev), q.to(dev)
    keys, vals = cd[0].transpose(1, 2), cd[1].transpose(1, 2)
    ops = _native.ops()
    y_plain = ops.attention(qd, keys, vals, 1.0 / np.sqrt(D))
    y_grp = ops.attention(qd, keys, vals, 1.0 / np.sqrt(D), P, G)
    assert torch.equal(y_grp, y_plain)
    ref = on.attention_f64(q.numpy(), cache[0].transpose(1, 2).numpy(), cache[1].transpose(1, 2).numpy())
    assert _rel(y_grp, ref) <= ATTN_TOL


@pytest.mark.parametrize("shape", [(6, 1, 4, 0, 23, 16, 40), (4, 2, 2, 50, 120, 64, 140), (1, 1, 2, 0, 2000, 128, 2100)],
                         ids=lambda s: "x".join(map(str, s)))
def test_decode_step_f64(dev, shape):
    """dg_decode_step in float64 (RoPE + QK-norm + append at pos, attention
    over 0 .. pos): the host- and device-position forms bit for bit equal to
    the two calls, the appended k within 16 ulps of the oracle's, y within the
    attention bar of float64 attention over the oracle's keys."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, G, H, P, pos, D, cap = shape
    groups = (B + G - 1) // G
    cache = torch.zeros((2, B, H, cap, D), dtype=torch.float64)
    if P:
        cache[:, :, :, :P] = _randn((groups, 2, H, P, D), 80 + D).repeat_interleave(G, dim=0)[:B].transpose(0, 1)
    cache[:, :, :, P:pos] = _randn((B, 2, H, pos - P, D), 81 + D).transpose(0, 1)
    q, k, v = (_randn((B, 1, H, D), 82 + D + i, 2.0) for i in range(3))
    table = precompute_freqs_cis(D, 2 * cap, 10000).double()
    scale = 1.0 / np.sqrt(D)
    prefix, group = (P, G) if G > 1 else (0, 1)
    ops = _native.ops()
    qd, kd, vd, td = q.to(dev), k.to(dev), v.to(dev), table.to(dev)

    # the two calls
    c2 = cache.to(dev)
    q_rot = torch.empty_like(qd)
    ops.rope_qknorm_append(qd, kd, vd, td[pos:pos + 1].view(1, 1, 1, D // 2, 2), q_rot,
                           c2[0, :, :, pos:pos + 1].transpose(1, 2), c2[1, :, :, pos:pos + 1].transpose(1, 2), True)
    y2 = ops.attention(q_rot, c2[0, :, :, :pos + 1].transpose(1, 2), c2[1, :, :, :pos + 1].transpose(1, 2), scale,
                       prefix, group)
    # the step, host position and device position
    for form in ("host", "device"):
        c1 = cache.to(dev)
        y1 = torch.empty_like(qd)
        if form == "host":
            _native.decode_step_(qd, kd, vd, td[pos].contiguous(), c1[0].transpose(1, 2), c1[1].transpose(1, 2), y1,
                                 scale, pos, prefix, group)
        else:
            p = torch.tensor([pos], dtype=torch.int32, device=dev)
            _native.decode_step_(qd, kd, vd, td, c1[0].transpose(1, 2), c1[1].transpose(1, 2), y1, scale, p,
                                 prefix, group)
        assert torch.equal(c1, c2), form
        assert torch.equal(y1, y2), form

    fc = np.broadcast_to(table[pos].numpy(), (B, 1, H, D // 2, 2))
    exp_q = on.rms_norm_f64(on.rope_f64(q.numpy(), fc))
    exp_k = on.rms_norm_f64(on.rope_f64(k.numpy(), fc))
    got_k = c2[0, :, :, pos:pos + 1].transpose(1, 2).cpu().numpy()
    assert np.abs(got_k - exp_k).max() <= 16 * EPS * np.abs(exp_k).max()
    keys = cache[0, :, :, :pos + 1].transpose(1, 2).numpy().copy()
    keys[:, pos:pos + 1] = exp_k
    vals = cache[1, :, :, :pos + 1].transpose(1, 2).numpy().copy()
    vals[:, pos:pos + 1] = v.numpy()
    assert _rel(y2, on.attention_f64(exp_q, keys, vals)) <= ATTN_TOL


# ------------------------------------------------------------------ row kernels around the attention


def test_row_kernels_f64(dev):
    """dg_attn_res_norm, dg_gate, dg_swiglu (alpha 1.702, not an fp32 value)
    and dg_softcap on float64 rows against the reference's torch formulas in
    float64 on the CPU (block.py:10-44 + rms_norm.py, mha.py:84,
    swi_glu.py:11-19, gpt.py:182-186)."""
    from diff_gpt import _native

    ops = _native.ops()
    M, C = 70, 96
    srcs = [_randn((M, C), 60 + i, 2.0) for i in range(5)]
    w = _randn((1, C), 66)
    got = ops.attn_res_norm([s.to(dev) for s in srcs], w.to(dev))
    exp = tr.rms(tr.attn_res(tuple(srcs[:-1]), srcs[-1], w)).numpy()
    assert np.abs(got.cpu().numpy() - exp).max() <= 64 * EPS * np.abs(exp).max()

    y, g = _randn((M, C), 67), _randn((M, C), 68, 3.0)
    yd = y.to(dev)
    ops.gate_(yd, g.to(dev))
    exp = (y * torch.sigmoid(g)).numpy()
    assert np.abs(yd.cpu().numpy() - exp).max() <= 16 * EPS * np.abs(exp).max()

    x = _randn((M, 2 * C), 69, 4.0)
    got = ops.swiglu(x.to(dev), 1.702, 7.0)
    gl, ln = x[:, ::2].clamp(max=7.0), x[:, 1::2].clamp(min=-7.0, max=7.0)
    exp = (gl * torch.sigmoid(1.702 * gl) * (ln + 1)).numpy()
    assert np.abs(got.cpu().numpy() - exp).max() <= 16 * EPS * np.abs(exp).max()

    z = _randn((M, 300), 70, 40.0)
    zd = z.to(dev)
    ops.softcap_(zd, 15.0)
    exp = (15.0 * torch.tanh(z / 15.0)).numpy()
    assert np.abs(zd.cpu().numpy() - exp).max() <= 16 * EPS * np.abs(exp).max()


def test_copy4d_f64_exact(dev):
    from diff_gpt import _native

    src = _randn((3, 5, 7, 9), 71)
    dst = torch.zeros((3, 9, 5, 7), dtype=torch.float64, device=dev).permute(0, 2, 3, 1)
    _native.ops().copy4d(src.to(dev), dst)
    assert torch.equal(dst.cpu(), src)


# ------------------------------------------------------------------ the model


def test_gpt_double_matches_oracle(dev):
    """GPT(...).double(): a prefill of 4 prompts of 40 ids (causal branch),
    a chunked prefill of 6 more ids (chunk branch), then 8 teacher-forced
    greedy decode steps; every step's logits within 1e-10 * max|ref| of the
    oracle's float64 forward and the argmax equal to its token wherever the
    top-2 margin exceeds twice that bar."""
    from diff_gpt.model.gpt import GPT
    from diff_gpt.model.kv_cache import KVCache

    torch.manual_seed(3)
    kw = dict(vocab_size=128, n_embd=64, block_size=64, n_head=4, n_layer=3)
    model = GPT(use_checkpoint=False, attn_res_layers_per_block=2, **kw).double().to(dev).eval()
    assert model.freqs_cis.dtype == torch.float64
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(attn_res_layers_per_block=2, **kw)
    prompts = torch.randint(0, 128, (4, 46), generator=torch.Generator().manual_seed(9))
    table = model.freqs_cis.cpu()
    ref_cache = tr.RefCache(4, 4, 64, 16, 3)
    kv = KVCache(batch_size=4, num_heads=4, seq_len=64, head_dim=16, num_layers=3)
    with torch.no_grad():
        for lo, hi in ((0, 40), (40, 46)):
            ref = tr.forward(params, cfg, prompts[:, lo:hi], ref_cache, table)
            got = model(prompts[:, lo:hi].to(dev), kv_cache=kv)[0]
            assert got.dtype == torch.float64
            err = (got.cpu() - ref).abs().max().item() / ref.abs().max().item()
            assert err <= MODEL_TOL, (lo, err)
        logits = got[:, -1]
        ref = ref[:, -1]
        for s in range(8):
            bar = MODEL_TOL * ref.abs().max().item()
            assert (logits.cpu() - ref).abs().max().item() <= bar, s
            tok = ref.argmax(-1)
            top2 = ref.topk(2, dim=-1).values
            clear = (top2[:, 0] - top2[:, 1]) > 2 * bar
            assert torch.equal(logits.argmax(-1).cpu()[clear], tok[clear])
            ref = tr.forward(params, cfg, tok[:, None], ref_cache, table)[:, -1]
            logits = model(tok[:, None].to(dev), kv_cache=kv)[0][:, -1]


def test_engine_double_graph_equals_eager(dev):
    """The Engine's captured decode step (device-read position) on a float64
    model gives the ids of an eager greedy loop over the same model."""
    from diff_gpt.model.engine import Engine
    from diff_gpt.model.gpt import GPT
    from diff_gpt.model.kv_cache import KVCache

    torch.manual_seed(4)
    model = GPT(vocab_size=128, n_embd=64, block_size=48, n_head=4, n_layer=2, use_checkpoint=False)
    model = model.double().to(dev).eval()
    prompt = [3, 17, 42, 8, 91, 5]
    greedy = lambda logits, rng: torch.argmax(logits, dim=-1, keepdim=True)  # noqa: E731
    rows, _ = Engine(model).generate_batch(tokens=prompt, num_samples=3, max_tokens=12, sampler=greedy)
    kv = KVCache(batch_size=1, num_heads=4, seq_len=len(prompt) + 12, head_dim=16, num_layers=2)
    ids = list(prompt)
    with torch.no_grad():
        logits = model(torch.tensor([prompt], device=dev), kv_cache=kv)[0][:, -1]
        for _ in range(12):
            nxt = int(logits.argmax(-1))
            ids.append(nxt)
            logits = model(torch.tensor([[nxt]], device=dev), kv_cache=kv)[0][:, -1]
    assert all(r == ids for r in rows)


def _random_f64_attn(seed, n):
    """Seeded (B, H, Tq, Tk, D): decode, causal and chunked, D even up to 1024."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = 2 * int(rng.integers(1, 513))
        B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        Tk = int(rng.integers(1, 700))
        kind = rng.integers(0, 3)
        Tq = 1 if kind == 0 else Tk if kind == 1 else int(rng.integers(1, Tk + 1))
        out.append((B, H, Tq, Tk, D))
    return out


@pytest.mark.parametrize("shape", _random_f64_attn(64, 10), ids=lambda s: "x".join(map(str, s)))
def test_attention_f64_random_shapes(dev, shape):
    """dg_attention in float64 at seeded random shapes against float64 brute force."""
    test_attention_f64(dev, shape)


@pytest.mark.parametrize("seed", [5, 6, 7])
def test_rope_f64_random_shapes(dev, seed):
    """Seeded random (B, T, H, D) rotations in float64 with a float64 table:
    bit-exact against the oracle."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    rng = np.random.default_rng(seed)
    B, T, H = (int(x) for x in rng.integers(1, 9, size=3))
    D = 2 * int(rng.integers(1, 513))
    pos = int(rng.integers(0, 100))
    x = _randn((B, T, H, D), seed, 2.0)
    fc = precompute_freqs_cis(D, pos + T, 10000).double()[pos:pos + T].view(1, T, 1, D // 2, 2)
    out = torch.empty((B, T, H, D), dtype=torch.float64, device=dev)
    _native.ops().rope_qknorm_append(x.to(dev), None, None, fc.to(dev), out, None, None, False)
    exp = on.rope_f64(x.numpy(), np.broadcast_to(fc.numpy(), (B, T, H, D // 2, 2)))
    assert np.array_equal(out.cpu().numpy().view(np.uint64), exp.view(np.uint64))
