"""The decode-step neighbour kernels (dg_block.hip) through the C-ABI, against
the oracle's torch-on-CPU restatement on the same inputs.

Bars: fp32 max-abs error <= 1e-5 * max|ref|,
bf16 and fp16 within 2e-2 * max|ref|; the one-source Block-AttnRes is dg_rms_norm bit
for bit (the softmax of one score is 1)."""

import numpy as np
import pytest
import torch

from oracle import torch_ref as tr

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 1e-5, "bf16": 2e-2, "f16": 2e-2}


def _randn(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(TDT[dtype])


def _rel(got: torch.Tensor, ref: torch.Tensor) -> float:
    g, r = got.double().cpu(), ref.double()
    return ((g - r).abs().max() / r.abs().max()).item()


RES = [  # (rows, C, sources)
    (6400, 64, 3),    # cfg1 decode, layer 0 MLP mixture (x, x, a0)
    (6400, 64, 4),
    (37, 64, 7),      # ragged row count
    (512, 512, 10),   # cfg3 width, eight layers deep
    (5, 1024, 5),     # cfg4 width
    (9, 48, 3),       # C not a power of two
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", RES, ids=lambda s: "x".join(map(str, s)))
def test_attn_res_norm_matches_reference(dev, dtype, shape):
    from diff_gpt import _native

    M, C, n = shape
    srcs = [_randn((M, C), 100 + i, dtype, 1.0 + 0.5 * i) for i in range(n)]
    w = _randn((1, C), 7, dtype, 0.5)
    got = _native.ops().attn_res_norm([s.to(dev) for s in srcs], w.to(dev))
    ref = tr.rms(tr.attn_res(tuple(srcs[:-1]), srcs[-1], w))
    assert got.dtype == ref.dtype and got.shape == ref.shape
    assert _rel(got, ref) <= TOL[dtype]


def _random_res(seed, n):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 7000)), int(rng.choice([16, 32, 48, 64, 96, 128, 256, 512, 1024])),
             int(rng.integers(2, 13))) for _ in range(n)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_res(17, 8), ids=lambda s: "x".join(map(str, s)))
def test_attn_res_norm_random_shapes(dev, dtype, shape):
    """Seeded random (rows, width, sources) through the same check."""
    test_attn_res_norm_matches_reference(dev, dtype, shape)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_attn_res_norm_one_source_is_rms_norm(dev, dtype):
    from diff_gpt import _native

    x = _randn((300, 64), 3, dtype, 3.0).to(dev)
    w = _randn((1, 64), 4, dtype).to(dev)
    a = _native.ops().attn_res_norm([x], w)
    b = _native.ops().rms_norm(x)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("C,n", [(512, 9), (1024, 5), (256, 3), (1000, 13), (2048, 2)])
def test_attn_res_norm_split_rows_equal_single_row_kernel(dev, dtype, C, n):
    """Up to 4096 wide rows go one row per workgroup of four waves (sources
    scored and columns summed in parallel); more rows go one row per wave.
    Both give the same bits: 4100 rows in one launch against their first 37
    rows and their last 512 in launches of their own."""
    from diff_gpt import _native

    M = 4100
    srcs = [_randn((M, C), 200 + i, dtype, 1.0 + 0.3 * i).to(dev) for i in range(n)]
    w = _randn((1, C), 8, dtype, 0.5).to(dev)
    ops = _native.ops()
    full = ops.attn_res_norm(srcs, w)
    for sl in (slice(0, 37), slice(M - 512, M)):
        part = ops.attn_res_norm([s[sl] for s in srcs], w)
        assert torch.equal(part, full[sl])
    one = ops.attn_res_norm([srcs[0][:64]], w)
    assert torch.equal(one, ops.rms_norm(srcs[0][:64]))


def test_attn_res_norm_strided_sources(dev):
    """Sources that are column slices of wider rows (row stride > C)."""
    from diff_gpt import _native

    wide = _randn((50, 3, 128), 11, "f32").to(dev)
    srcs = [wide[:, i, 32:96] for i in range(3)]
    w = _randn((1, 64), 12, "f32").to(dev)
    got = _native.ops().attn_res_norm(srcs, w)
    ref = tr.rms(tr.attn_res(tuple(s.cpu() for s in srcs[:-1]), srcs[-1].cpu(), w.cpu()))
    assert _rel(got, ref) <= TOL["f32"]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_gate_matches_reference(dev, dtype):
    from diff_gpt import _native

    y = _randn((6400, 64), 21, dtype)
    wide = _randn((6400, 256), 22, dtype, 3.0)
    g = wide[:, 192:]  # the g slice of a fused projection output
    yd = y.to(dev)
    _native.ops().gate_(yd, wide.to(dev)[:, 192:])
    ref = y * torch.sigmoid(g)
    assert _rel(yd, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows", [6400, 3])
def test_swiglu_matches_reference(dev, dtype, rows):
    from diff_gpt import _native

    alpha, limit = 1.702, 7.0
    h = _randn((rows, 256), 31 + rows, dtype, 5.0)  # crosses the clamp limits
    got = _native.ops().swiglu(h.to(dev), alpha, limit)
    gl = h[..., ::2].clamp(max=limit)
    ln = h[..., 1::2].clamp(min=-limit, max=limit)
    ref = gl * torch.sigmoid(alpha * gl) * (ln + 1)
    assert got.shape == (rows, 128)
    assert _rel(got, ref) <= TOL[dtype]


@pytest.mark.parametrize("pair,alpha,limit,expected", [
    # the reference's known answers (tests/diff_gpt/model/test_swi_glu.py:21-102),
    # the sigmoid written out: y = g * 1 / (1 + exp(-alpha * g)) * (l + 1)
    ((1.0, 2.0), 2.0, 100.0, 1.0 / (1.0 + np.exp(-2.0)) * 3.0),      # no clamp
    ((10.0, 10.0), 1.0, 5.0, 5.0 / (1.0 + np.exp(-5.0)) * 6.0),      # both halves clamped above
    ((1.0, -10.0), 1.0, 5.0, 1.0 / (1.0 + np.exp(-1.0)) * -4.0),     # linear half clamped below
    ((-10.0, 0.0), 1.0, 5.0, -10.0 / (1.0 + np.exp(10.0)) * 1.0),    # gate half has no lower clamp
])
def test_swiglu_kernel_known_answers(dev, pair, alpha, limit, expected):
    """dg_swiglu on one (gate, linear) pair, fp32, at the reference's known
    answers: within fp32 rounding of the closed form."""
    from diff_gpt import _native

    got = _native.ops().swiglu(torch.tensor([list(pair)], device=dev), alpha, limit)
    assert got.shape == (1, 1)
    assert abs(got.item() - expected) <= 1e-6 * max(1.0, abs(expected))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_softcap_matches_reference(dev, dtype):
    from diff_gpt import _native

    x = _randn((6400, 256), 41, dtype, 20.0)
    xd = x.to(dev)
    _native.ops().softcap_(xd, 15.0)
    ref = 15.0 * torch.tanh(x / 15.0)
    assert _rel(xd, ref) <= TOL[dtype]
    assert xd.float().abs().max().item() <= 15.0


def test_gpt_forward_uses_one_projection_gemm_and_matches_reference(dev):
    """GPT.forward with the fused neighbours against the oracle forward on the
    same weights (fp32, prefill of 2 x 24 tokens)."""
    from diff_gpt.model.gpt import GPT

    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=64, n_head=4, n_layer=3,
                use_checkpoint=False).eval()
    p = {k: v.detach().clone() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=64, block_size=64, n_head=4, n_layer=3)
    idx = torch.randint(0, 256, (2, 24), generator=torch.Generator().manual_seed(5))
    model = model.to(dev)
    with torch.inference_mode():
        got, _ = model(idx.to(dev))
        ref = tr.forward(p, cfg, idx)
    assert _rel(got, ref) <= TOL["f32"]
    # the four projection weights are views of the one GEMM operand: an update
    # through .data (which leaves _version alone) reaches the next forward
    sa = model.blocks[0].sa
    w0 = sa._projection_weight()
    assert sa._projection_weight() is w0
    sa.c_g.weight.data.mul_(2.0)
    sa.c_q.weight.data.copy_(sa.c_q.weight.data * 0.5)
    assert sa._projection_weight() is w0
    assert np.array_equal(w0[192:].cpu().numpy(), sa.c_g.weight.detach().cpu().numpy())
    p["blocks.0.sa.c_g.weight"] *= 2.0
    p["blocks.0.sa.c_q.weight"] *= 0.5
    with torch.inference_mode():
        got, _ = model(idx.to(dev))
        ref = tr.forward(p, cfg, idx)
    assert _rel(got, ref) <= TOL["f32"]


@pytest.mark.parametrize("C,nsrc", [(64, 36), (2304, 3)], ids=["36_sources", "width_2304"])
def test_attn_res_norm_beyond_kernel_limits(dev, C, nsrc):
    """More than 32 sources or more than 2048 columns exceed dg_attn_res_norm:
    block.attn_res_norm then mixes with device torch ops and normalises with
    dg_rms_norm, still within the fp32 bar of the oracle."""
    from diff_gpt.model.block import attn_res_norm

    srcs = [_randn((40, C), 200 + i, "f32", 1.0 + 0.1 * i) for i in range(nsrc)]
    proj = torch.nn.Linear(C, 1, bias=False)
    with torch.no_grad():
        proj.weight.copy_(_randn((1, C), 9, "f32", 0.5))
    with torch.inference_mode():
        got = attn_res_norm(tuple(s.to(dev) for s in srcs[:-1]), srcs[-1].to(dev), proj.to(dev))
        # the oracle in float64: the exact function of these fp32 inputs (at
        # 2304 columns the CPU's own fp32 dot products sit ~1e-5 from it)
        ref = tr.rms(tr.attn_res(tuple(s.double() for s in srcs[:-1]), srcs[-1].double(),
                                 proj.weight.detach().cpu().double()))
    assert _rel(got, ref) <= TOL["f32"]


# the wide model's fp32 GEMMs (K = 2304 and 9216) sum in another order than
# the CPU's: about 1e-5 of max|logit| after two layers
@pytest.mark.parametrize("n_embd,n_head,n_layer,bar", [(32, 2, 33, 1e-5), (2304, 18, 2, 5e-5)],
                         ids=["deep", "wide"])
def test_gpt_beyond_attn_res_kernel_limits(dev, n_embd, n_head, n_layer, bar):
    """33 layers (the last sub-layers mix up to 36 sources) and n_embd 2304
    exceed dg_attn_res_norm's 32 sources / 2048 columns: GPT.forward takes the
    fallback mixture and still matches the oracle."""
    from diff_gpt.model.gpt import GPT

    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=n_embd, block_size=32, n_head=n_head, n_layer=n_layer,
                use_checkpoint=False).eval()
    p = {k: v.detach().clone() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=n_embd, block_size=32, n_head=n_head, n_layer=n_layer)
    idx = torch.randint(0, 256, (2, 12), generator=torch.Generator().manual_seed(7))
    model = model.to(dev)
    with torch.inference_mode():
        got, _ = model(idx.to(dev))
        ref = tr.forward(p, cfg, idx)
    assert _rel(got, ref) <= bar


LM_HEAD = [  # (rows, C, V)
    (6400, 64, 256),   # cfg1 decode step
    (37, 512, 256),    # cfg3 width, ragged rows
    (5, 1024, 256),    # cfg4 width
    (48, 64, 1024),    # widest vocabulary taken
    (16, 128, 64),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("cap", [15.0, 0.0], ids=["softcap", "nocap"])
@pytest.mark.parametrize("shape", LM_HEAD, ids=lambda s: "x".join(map(str, s)))
def test_lm_head_matches_linear_softcap_argmax(dev, dtype, cap, shape):
    """dg_lm_head against F.linear + softcap on the same rows (north-star
    bars), and its argmax equal to torch.argmax of the logits it stored."""
    from diff_gpt import _native

    M, C, V = shape
    x = tr.rms(_randn((M, C), 90 + C, dtype, 2.0))
    w = _randn((V, C), 91 + V, dtype, 1.0)
    logits = torch.empty((M, V), dtype=TDT[dtype], device=dev)
    ids = torch.full((M,), -1, dtype=torch.int64, device=dev)
    assert _native.lm_head_(x.to(dev), w.to(dev), cap, logits, ids)
    ref = x.float() @ w.float().t()
    ref = ref.to(TDT[dtype]).float()
    if cap > 0:
        ref = cap * torch.tanh(ref / cap)
    assert _rel(logits, ref) <= TOL[dtype]
    assert torch.equal(ids, torch.argmax(logits, dim=-1))


def _random_lm_heads(seed, n):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 3000)), int(rng.choice([64, 128, 192, 320, 512, 1024])),
             int(rng.choice([64, 128, 256, 512, 1024]))) for _ in range(n)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_lm_heads(31, 8), ids=lambda s: "x".join(map(str, s)))
def test_lm_head_random_shapes(dev, dtype, shape):
    """Seeded random (rows, width, vocabulary) within the kernel's range, with
    the softcap: logits within the bars, argmax equal to torch.argmax."""
    test_lm_head_matches_linear_softcap_argmax(dev, dtype, 15.0, shape)


def test_lm_head_argmax_first_maximum_wins(dev):
    """Equal maxima (rows of the table repeated) resolve to the first entry,
    as torch.argmax does, including across the four waves' quarters."""
    from diff_gpt import _native

    M, C, V = 32, 64, 256
    x = _randn((M, C), 5, "f32").to(dev)
    base = _randn((1, C), 6, "f32")
    w = _randn((V, C), 7, "f32") * 0.01
    for e in (3, 64, 130, 250):  # the same best row in several quarters
        w[e] = base[0]
    w = w.to(dev)
    x = base.repeat(M, 1).to(dev)  # every row's maximum is at entries 3, 64, 130, 250
    logits = torch.empty((M, V), device=dev)
    ids = torch.empty((M,), dtype=torch.int64, device=dev)
    assert _native.lm_head_(x, w, 15.0, logits, ids)
    assert bool((ids == 3).all())
    assert torch.equal(ids, torch.argmax(logits, dim=-1))


@pytest.mark.parametrize("shape", [(8, 48, 256), (8, 64, 300), (8, 64, 192)], ids=lambda s: "x".join(map(str, s)))
def test_lm_head_unsupported_shapes_do_nothing(dev, shape):
    from diff_gpt import _native

    M, C, V = shape
    logits = torch.full((M, V), 7.0, device=dev)
    assert not _native.lm_head_(torch.ones((M, C), device=dev), torch.ones((V, C), device=dev), 15.0, logits)
    assert bool((logits == 7.0).all())


def test_gpt_greedy_generate_uses_fused_argmax(dev, monkeypatch):
    """GPT.generate with TemperatureSampler(0) takes the argmax from the
    lm_head launch; the tokens equal those of the unfused path (F.linear +
    softcap + torch.argmax), which forcing the fallback gives."""
    from diff_gpt import _native
    from diff_gpt.model.gpt import GPT
    from diff_gpt.sampler.temperature import TemperatureSampler

    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=32, n_head=4, n_layer=2, use_checkpoint=False).to(dev).eval()
    idx = torch.randint(0, 256, (3, 5), generator=torch.Generator().manual_seed(1)).to(dev)
    with torch.inference_mode():
        fused = model.generate(idx, 12, TemperatureSampler(0))
    real = _native.lm_head_
    monkeypatch.setattr(_native, "lm_head_", lambda *a, **k: False)
    with torch.inference_mode():
        plain = model.generate(idx, 12, TemperatureSampler(0))
    monkeypatch.setattr(_native, "lm_head_", real)
    assert torch.equal(fused, plain)


# ------------------------------------------------------------------ a layer in three launches

LAYER = [  # (rows, C, committed blocks, commits its input)
    (6400, 64, 2, True),    # cfg1 decode step, layer 0: blocks (x, x)
    (6400, 64, 3, True),    # layer 1
    (37, 64, 5, False),     # ragged rows; a layer inside a block: partial_in + attention output
    (100, 128, 3, True),    # n_embd 128
    (17, 128, 1, False),
    (1, 64, 30, True),      # one row; 31 mixture sources
]
ALPHA, LIMIT = 1.702, 7.0


def _layer_case(M, C, nblk, dtype, seed):
    """Blocks, partial_in, the attention output y, the gate logits g (a column
    slice of a wider projection row, as in the model) and the layer's weights,
    with a scale that keeps every stage O(1)."""
    blocks = [_randn((M, C), seed + i, dtype, 1.0 + 0.3 * i) for i in range(nblk)]
    pin = _randn((M, C), seed + 50, dtype)
    y = _randn((M, C), seed + 51, dtype)
    qkvg = _randn((M, 4 * C), seed + 52, dtype, 2.0)
    w = {
        "proj": _randn((C, C), seed + 53, dtype, C ** -0.5),
        "mix_mlp": _randn((1, C), seed + 55, dtype, 0.5),
        "up": _randn((4 * C, C), seed + 57, dtype, 3.0 * C ** -0.5),
        "down": _randn((C, 2 * C), seed + 58, dtype, (2 * C) ** -0.5),
    }
    return blocks, pin, y, qkvg, w


def _swiglu64(h):
    gl = h[..., ::2].clamp(max=LIMIT)
    ln = h[..., 1::2].clamp(min=-LIMIT, max=LIMIT)
    return gl * torch.sigmoid(ALPHA * gl) * (ln + 1)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", LAYER, ids=lambda s: "x".join(map(str, s)))
def test_block_out_matches_reference(dev, dtype, shape):
    """dg_block_out (gate, c_proj, the partial sum, the MLP's mixture and norm,
    FFN up, SwiGLU, FFN down, residual) against the oracle's functions
    evaluated in float64 on the same inputs (fp32 at 1e-5; bf16 / fp16 at
    2e-2, or 1.5x the reference's own evaluation in that dtype where its
    rounding alone exceeds it), and against the separate launches it replaces
    on the device at the dtype's bar."""
    from diff_gpt import _native
    from diff_gpt.model.block import attn_res_norm

    M, C, nblk, committed = shape
    blocks, pin, y, qkvg, w = _layer_case(M, C, nblk, dtype, 300 + C + nblk)
    g = qkvg[:, 3 * C:]
    d = lambda t: t.to(dev)  # noqa: E731
    out = torch.empty((M, C), dtype=TDT[dtype], device=dev)
    assert _native.block_out_(d(y), d(qkvg)[:, 3 * C:], d(w["proj"]), None if committed else d(pin),
                              [d(b) for b in blocks], d(w["mix_mlp"]), d(w["up"]), d(w["down"]), ALPHA, LIMIT, out)
    # the oracle, float64
    f = {k: v.double() for k, v in w.items()}
    a = (y.double() * torch.sigmoid(g.double())) @ f["proj"].T
    pm = a if committed else pin.double() + a
    xn = tr.rms(tr.attn_res(tuple(b.double() for b in blocks), pm, f["mix_mlp"]))
    ref = pm + _swiglu64(xn @ f["up"].T) @ f["down"].T
    err = _rel(out, ref)
    # the separate launches on the device (the unfused path)
    with torch.inference_mode():
        ya = d(y).clone()
        _native.ops().gate_(ya, d(qkvg)[:, 3 * C:])
        a2 = torch.nn.functional.linear(ya, d(w["proj"]))
        pm2 = a2 if committed else d(pin) + a2
        xn2 = attn_res_norm(tuple(d(b) for b in blocks), pm2, _Proj(d(w["mix_mlp"])))
        h2 = _native.ops().swiglu(torch.nn.functional.linear(xn2, d(w["up"])), ALPHA, LIMIT)
        sep = pm2 + torch.nn.functional.linear(h2, d(w["down"]))
    # the reference's own evaluation in the dtype (torch on the CPU, each op
    # rounding as it returns): through seven stages bf16 / fp16 rounding alone
    # can move the result by about the north-star bar, so the bar against
    # float64 is that deviation x 1.5 where it exceeds the bar
    a3 = (y * torch.sigmoid(g)) @ w["proj"].T
    pm3 = a3 if committed else pin + a3
    xn3 = tr.rms(tr.attn_res(tuple(blocks), pm3, w["mix_mlp"]))
    own = _rel(pm3 + _swiglu64(xn3 @ w["up"].T) @ w["down"].T, ref)
    print(f"block_out {shape} {dtype}: |fused - f64| {err:.3g}, |unfused - f64| {_rel(sep, ref):.3g}, "
          f"|reference {dtype} - f64| {own:.3g}, |fused - unfused| {_rel(out, sep.double().cpu()):.3g} "
          f"(x max|ref|)", flush=True)
    assert err <= max(TOL[dtype], 1.5 * own), (err, own)
    assert _rel(out, sep.double().cpu()) <= TOL[dtype]


class _Proj:
    """The .weight holder block.attn_res_norm reads its pseudo-query from."""

    def __init__(self, w):
        self.weight = w


@pytest.mark.parametrize("C", [32, 96, 256])
def test_block_out_declines_other_widths(dev, C):
    """n_embd other than 64 or 128: dg_block_out returns False and writes
    nothing (the model then makes the separate launches)."""
    from diff_gpt import _native

    M = 20
    blocks, pin, y, qkvg, w = _layer_case(M, C, 2, "f32", 7)
    d = lambda t: t.to(dev)  # noqa: E731
    out = torch.full((M, C), 5.0, device=dev)
    assert not _native.block_out_(d(y), d(qkvg)[:, 3 * C:], d(w["proj"]), None, [d(b) for b in blocks],
                                  d(w["mix_mlp"]), d(w["up"]), d(w["down"]), ALPHA, LIMIT, out)
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("layers_per_block", [1, 2])
def test_gpt_layers_with_fused_block_out_match_separate_launches(dev, dtype, layers_per_block, monkeypatch):
    """GPT.forward at n_embd 64 ends each layer with one dg_block_out launch;
    with it declined it makes the separate launches.  The logits of a prefill
    and a decode step agree within the dtype's bar, and the fp32 ones with the
    oracle forward within 1e-5 (layers_per_block 2: half the layers add their
    attention output to the partial sum they were given)."""
    from diff_gpt import _native
    from diff_gpt.model.gpt import GPT
    from diff_gpt.model.kv_cache import KVCache

    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=64, n_head=4, n_layer=4, use_checkpoint=False,
                attn_res_layers_per_block=layers_per_block).eval()
    p = {k: v.detach().clone() for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=64, block_size=64, n_head=4, n_layer=4,
                         attn_res_layers_per_block=layers_per_block)
    model = model.to(dev).to(TDT[dtype])
    idx = torch.randint(0, 256, (3, 20), generator=torch.Generator().manual_seed(2))
    calls = [0]
    real_out = _native.block_out_

    def counted(*a, **k):
        calls[0] += 1
        return real_out(*a, **k)

    def run():
        kv = KVCache(batch_size=3, num_heads=4, seq_len=21, head_dim=16, num_layers=4)
        with torch.inference_mode():
            first = model(idx.to(dev), kv_cache=kv)[0][:, -1]
            step = model(first.argmax(-1, keepdim=True), kv_cache=kv)[0][:, -1]
        return first.float().cpu(), step.float().cpu()

    monkeypatch.setattr(_native, "block_out_", counted)
    fused = run()
    assert calls[0] == 8  # 4 layers x (prefill, step)
    monkeypatch.setattr(_native, "block_out_", lambda *a, **k: False)
    separate = run()
    for f_, s_ in zip(fused, separate):
        assert _rel(f_, s_.double()) <= TOL[dtype]
    if dtype == "f32":
        with torch.no_grad():
            ref = tr.forward(p, cfg, idx)[:, -1]
        assert _rel(fused[0], ref) <= 1e-5


EMB = [  # (rows, C, vocab)
    (6400, 64, 256),  # cfg1 decode step: one token per trajectory
    (37, 64, 96),     # ragged row count
    (512, 512, 1024),
    (5, 1024, 64),
    (9, 48, 33),      # C not a power of two (no vector access)
    (3, 8192, 16),    # widest row
    (4, 1, 8),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", EMB, ids=lambda s: "x".join(map(str, s)))
def test_embed_norm_is_embedding_then_rms_norm_bit_for_bit(dev, dtype, shape):
    """dg_embed_norm writes rms_norm(table[ids]) and rms_norm of that row as
    stored: the bits of nn.Embedding followed by dg_rms_norm twice, and the
    fp32 oracle within the dtype's bar."""
    from diff_gpt import _native

    M, C, V = shape
    table = _randn((V, C), 11, dtype, 0.7)
    ids = torch.randint(0, V, (M,), generator=torch.Generator().manual_seed(3))
    t, i = table.to(dev), ids.to(dev)
    x = torch.empty((M, C), dtype=t.dtype, device=dev)
    xn = torch.empty_like(x)
    assert _native.embed_norm_(i, t, x, xn)
    sep_x = _native.ops().rms_norm(torch.nn.functional.embedding(i, t))
    sep_xn = _native.ops().rms_norm(sep_x)
    assert torch.equal(x, sep_x) and torch.equal(xn, sep_xn)
    ref = tr.rms(table.float()[ids])
    assert _rel(x, ref) <= TOL[dtype]
    assert _rel(xn, tr.rms(x.float().cpu())) <= TOL[dtype]
    # without the second output
    x1 = torch.empty_like(x)
    assert _native.embed_norm_(i, t, x1, None)
    assert torch.equal(x1, sep_x)


def test_embed_norm_bad_ids_give_nan_rows(dev):
    """An id outside [0, V) reads nothing outside the table: its rows are NaN,
    the other rows are those of valid ids."""
    from diff_gpt import _native

    table = _randn((16, 64), 5, "f32").to(dev)
    ids = torch.tensor([3, -1, 16, 15, 1 << 40, 0], device=dev)
    x = torch.empty((6, 64), device=dev)
    xn = torch.empty_like(x)
    assert _native.embed_norm_(ids, table, x, xn)
    bad = torch.tensor([False, True, True, False, True, False])
    xc, xnc = x.cpu(), xn.cpu()
    assert bool(xc[bad].isnan().all()) and bool(xnc[bad].isnan().all())
    good = ids.cpu()[~bad]
    assert torch.equal(xc[~bad], _native.ops().rms_norm(table[good.to(dev)]).cpu())


def test_embed_norm_declines_fp64_and_strided_tables(dev):
    from diff_gpt import _native

    ids = torch.zeros(4, dtype=torch.int64, device=dev)
    t64 = torch.randn(8, 64, dtype=torch.float64, device=dev)
    x64 = torch.full((4, 64), 5.0, dtype=torch.float64, device=dev)
    assert not _native.embed_norm_(ids, t64, x64, None)
    tT = torch.randn(64, 8, device=dev).t()
    x = torch.full((4, 64), 5.0, device=dev)
    assert not _native.embed_norm_(ids, tT, x, None)
    torch.cuda.synchronize()
    assert bool((x64 == 5.0).all()) and bool((x == 5.0).all())


def test_gpt_embedding_launch_feeds_layer_zero(dev, monkeypatch):
    """GPT.forward gathers and normalises the embedding and layer 0's
    attention input in one dg_embed_norm launch; with it declined (nn.Embedding,
    then the RMSNorm kernel and layer 0's own norm) the logits are equal."""
    from diff_gpt import _native
    from diff_gpt.model.gpt import GPT

    torch.manual_seed(0)
    model = GPT(vocab_size=128, n_embd=64, block_size=32, n_head=4, n_layer=2,
                use_checkpoint=False).eval().to(dev).to(torch.bfloat16)
    idx = torch.randint(0, 128, (3, 17), generator=torch.Generator().manual_seed(4)).to(dev)
    calls = [0]
    real = _native.embed_norm_

    def counted(*a, **k):
        calls[0] += 1
        return real(*a, **k)

    with torch.inference_mode():
        monkeypatch.setattr(_native, "embed_norm_", counted)
        fused = model(idx)[0]
        assert calls[0] == 1
        monkeypatch.setattr(_native, "embed_norm_", lambda *a, **k: False)
        separate = model(idx)[0]
    assert torch.equal(fused, separate)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", LAYER, ids=lambda s: "x".join(map(str, s)))
def test_block_out_norm_adds_the_head_norm_bit_for_bit(dev, dtype, shape):
    """dg_block_out_norm writes dg_block_out's output bits and rms_norm of
    them with dg_rms_norm's bits (the head's input after the last layer),
    including the rows of a partial last tile."""
    from diff_gpt import _native

    M, C, nblk, committed = shape
    blocks, pin, y, qkvg, w = _layer_case(M, C, nblk, dtype, 700 + C + nblk)
    d = lambda t: t.to(dev)  # noqa: E731
    args = (d(y), d(qkvg)[:, 3 * C:], d(w["proj"]), None if committed else d(pin), [d(b) for b in blocks],
            d(w["mix_mlp"]), d(w["up"]), d(w["down"]), ALPHA, LIMIT)
    out = torch.empty((M, C), dtype=TDT[dtype], device=dev)
    assert _native.block_out_(*args, out)
    out2 = torch.empty_like(out)
    xn = torch.full_like(out, 7.0)
    assert _native.block_out_(*args, out2, xn)
    assert torch.equal(out, out2)
    assert torch.equal(xn, _native.ops().rms_norm(out))
    assert _rel(xn, tr.rms(out.float().cpu())) <= TOL[dtype]


def test_gpt_head_norm_from_the_last_layer(dev, monkeypatch):
    """GPT.forward takes the head's RMSNorm from the last layer's
    dg_block_out_norm launch; with the fused layer declined (separate
    launches, then dg_rms_norm) the logits agree within the bf16 bar, and a
    forward with the head norm taken from dg_rms_norm instead gives equal
    logits."""
    from diff_gpt import _native
    from diff_gpt.model.gpt import GPT
    from diff_gpt.model.kv_cache import KVCache

    torch.manual_seed(0)
    model = GPT(vocab_size=128, n_embd=64, block_size=32, n_head=4, n_layer=3,
                use_checkpoint=False).eval().to(dev).to(torch.bfloat16)
    idx = torch.randint(0, 128, (3, 17), generator=torch.Generator().manual_seed(5)).to(dev)
    real = _native.block_out_
    seen = []

    def counted(*a, **k):
        seen.append(len(a) > 11 and a[11] is not None)
        return real(*a, **k)

    def without_norm(*a, **k):
        ok = real(*a[:11], **k)
        if ok and len(a) > 11 and a[11] is not None:
            _native.rms_norm_(a[10], a[11])
        return ok

    def run():
        kv = KVCache(batch_size=3, num_heads=4, seq_len=18, head_dim=16, num_layers=3)
        with torch.inference_mode():
            first = model(idx, kv_cache=kv)[0]
            step = model(first[:, -1].argmax(-1, keepdim=True), kv_cache=kv)[0]
            last = model(idx, _last_only=True)[0]
        return first, step, last

    monkeypatch.setattr(_native, "block_out_", counted)
    fused = run()
    assert seen == [False, False, True] * 3
    monkeypatch.setattr(_native, "block_out_", without_norm)
    same = run()
    for f_, s_ in zip(fused, same):
        assert torch.equal(f_, s_)
    monkeypatch.setattr(_native, "block_out_", lambda *a, **k: False)
    separate = run()
    for f_, s_ in zip(fused, separate):
        assert _rel(f_, s_.double().cpu()) <= TOL["bf16"]


DRAW = [(6400, 256), (37, 96), (5, 1), (3, 1000), (2, 64)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16", "f64"])
@pytest.mark.parametrize("shape", DRAW, ids=lambda s: "x".join(map(str, s)))
def test_draw_argmax_equals_torch_argmax_of_quotient(dev, dtype, shape):
    """dg_draw_argmax gives torch.argmax(probs / q, -1)'s ids on the device,
    with ties (repeated probabilities and variates), zeros, an infinite
    quotient and NaN rows planted."""
    from diff_gpt import _native

    M, V = shape
    dt = torch.float64 if dtype == "f64" else TDT[dtype]
    g = torch.Generator().manual_seed(9 + V)
    probs = torch.softmax(torch.randn((M, V), generator=g, dtype=torch.float64) * 2, -1)
    q = torch.empty((M, V), dtype=torch.float64).exponential_(1, generator=g)
    if V >= 4:
        probs[0, :4] = 0.25  # ties
        q[0, :4] = 1.0
        probs[1 % M, 2] = 0.0
        q[min(2, M - 1), 3] = 0.0  # an infinite quotient (or 0/0)
        probs[M - 1, V // 2] = float("nan")
        probs[M - 1, V - 1] = float("nan")
    p, qq = probs.to(dt).to(dev), q.to(dt).to(dev)
    ids = torch.empty((M, 1), dtype=torch.int64, device=dev)
    assert _native.draw_argmax_(p, qq, ids)
    assert torch.equal(ids, torch.argmax(p / qq, dim=-1, keepdim=True))
    # the oracle's statement on the host
    assert torch.equal(ids.cpu(), torch.argmax(p.cpu() / qq.cpu(), dim=-1, keepdim=True))


def test_temperature_sampler_draw_is_multinomial(dev):
    """The sampler's one-launch draw gives torch.multinomial's ids on the same
    generator state (its one-sample method) for a temperature-1 step."""
    from diff_gpt.sampler.temperature import TemperatureSampler

    logits = torch.randn((640, 256), generator=torch.Generator().manual_seed(3)).to(dev)
    s = TemperatureSampler(1.0)
    g1 = torch.Generator(device=dev)
    g1.manual_seed(11)
    got = s(logits, rng=g1)
    g2 = torch.Generator(device=dev)
    g2.manual_seed(11)
    ref = torch.multinomial(torch.softmax(logits, -1), 1, generator=g2)
    assert torch.equal(got, ref)
