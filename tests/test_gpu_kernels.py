"""Kernel parity on the GPU through the C-ABI (libdgattn via diff_gpt._native).

Bars:
  * RoPE / QK-norm / KV append: bit-exact against oracle.numerics (same
    canonical fp32 operation order); V and plain copies exact.
  * attention: fp32 max-abs error <= 1e-5 * max|ref|; bf16 / fp16 within
    2e-2 * max|ref| -- against float64 brute force on the same inputs.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import numerics as on

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 1e-5, "bf16": 2e-2, "f16": 2e-2}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().view(np.uint32)


def _randn(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(TDT[dtype])


# ------------------------------------------------------------------ RoPE + QK-norm + append


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [8, 16, 64, 128, 256, 12])
def test_rope_qknorm_append_bit_exact(dev, dtype, D):
    _rope_append_case(dev, dtype, 3, 5, 4, D, 7, 16)


def _random_rope_appends(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([8, 12, 16, 32, 48, 64, 128, 256]))
        B, T, H = int(rng.integers(1, 9)), int(rng.integers(1, 300)), int(rng.integers(1, 9))
        pos = int(rng.integers(0, 200))
        out.append((B, T, H, D, pos, pos + T + int(rng.integers(0, 30))))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_rope_appends(99, 10), ids=lambda s: "x".join(map(str, s)))
def test_rope_qknorm_append_random_shapes(dev, dtype, shape):
    """Seeded random (B, T, H, D, position, capacity): rotated and normalised
    q and k bit-exact against the oracle, v copied, the rest untouched."""
    _rope_append_case(dev, dtype, *shape)


@pytest.mark.parametrize("dtype,B,T,H,D", [("bf16", 33, 1000, 8, 64), ("f32", 9, 2000, 30, 16),
                                           ("f16", 11, 1500, 9, 128)])
def test_rope_qknorm_append_many_rows(dev, dtype, B, T, H, D):
    """Launches of at least 2048 workgroups of 4-row lane groups (a prefill's
    rows) take several rows per lane group, with a ragged last workgroup
    here: still bit-exact against the oracle."""
    _rope_append_case(dev, dtype, B, T, H, D, 3, T + 5)


def _rope_append_case(dev, dtype, B, T, H, D, pos, cap):
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    q = _randn((B, T, H, D), 10 + D, dtype, 2.0)
    k = _randn((B, T, H, D), 20 + D, dtype, 2.0)
    v = _randn((B, T, H, D), 30 + D, dtype)
    table = precompute_freqs_cis(D, max(64, cap), 10000).to(TDT[dtype])
    fc = table[pos:pos + T].view(1, T, 1, D // 2, 2)

    cache = torch.full((2, 2, B, H, cap, D), 7.0, dtype=TDT[dtype])
    layer = 1
    qd, kd, vd, fd = (t.to(dev) for t in (q, k, v, fc))
    cd = cache.to(dev)
    q_out = torch.empty_like(qd)
    k_dst = cd[layer, 0, :, :, pos:pos + T].transpose(1, 2)
    v_dst = cd[layer, 1, :, :, pos:pos + T].transpose(1, 2)
    _native.ops().rope_qknorm_append(qd, kd, vd, fd, q_out, k_dst, v_dst, True)
    torch.cuda.synchronize()

    fcn = fc.float().numpy()
    exp_q = on.rope_qknorm(q.float().numpy(), fcn, dtype)
    exp_k = on.rope_qknorm(k.float().numpy(), fcn, dtype)
    got = cd.cpu()
    assert np.array_equal(_bits(q_out), exp_q.view(np.uint32))
    assert np.array_equal(_bits(got[layer, 0, :, :, pos:pos + T].transpose(1, 2)),
                          exp_k.view(np.uint32))
    assert torch.equal(got[layer, 1, :, :, pos:pos + T].transpose(1, 2), v)
    # nothing outside the window was touched
    untouched = got.clone()
    untouched[layer, :, :, :, pos:pos + T] = 7.0
    assert (untouched == 7.0).all()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_rope_only_bit_exact_with_broadcast_table(dev, dtype):
    from diff_gpt.model.rope import apply_rotary_emb

    x = _randn((2, 4, 8, 10), 3, dtype)  # D = 10: not a power of two
    g = torch.Generator().manual_seed(4)
    th = torch.randn(1, 1, 8, 5, generator=g)
    fc = torch.stack([th.cos(), th.sin()], -1).to(TDT[dtype])
    out = apply_rotary_emb(x.to(dev), fc.to(dev))
    exp = on.rope(x.float().numpy(), np.broadcast_to(fc.float().numpy(), (2, 4, 8, 5, 2)), dtype)
    assert out.shape == x.shape and out.dtype == x.dtype
    assert np.array_equal(_bits(out), exp.view(np.uint32))


# ------------------------------------------------------------------ row RMSNorm


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("N", [5, 16, 64, 100, 1024, 4096])
def test_rms_norm_bit_exact(dev, dtype, N):
    from diff_gpt.model.rms_norm import rms_norm

    x = _randn((3, 37, N), N, dtype, 3.0)
    y = rms_norm(x.to(dev))
    exp = on.rms_norm(x.float().numpy(), dtype)
    assert y.dtype == x.dtype and y.shape == x.shape
    assert np.array_equal(_bits(y), exp.view(np.uint32))


# ------------------------------------------------------------------ attention


def _attention_case(dev, dtype, B, H, Tq, Tk, D, cache_layout, seed):
    from diff_gpt import _native

    q = _randn((B, Tq, H, D), seed, dtype)
    k = _randn((B, Tk, H, D), seed + 1, dtype)
    v = _randn((B, Tk, H, D), seed + 2, dtype)
    ref = on.attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy())
    if cache_layout:
        cap = Tk + 5
        kc = torch.zeros((B, H, cap, D), dtype=TDT[dtype], device=dev)
        vc = torch.zeros_like(kc)
        kc[:, :, :Tk] = k.transpose(1, 2).to(dev)
        vc[:, :, :Tk] = v.transpose(1, 2).to(dev)
        kd, vd = kc[:, :, :Tk].transpose(1, 2), vc[:, :, :Tk].transpose(1, 2)
    else:
        kd, vd = k.to(dev), v.to(dev)
    y = _native.ops().attention(q.to(dev), kd, vd, 1.0 / np.sqrt(D))
    got = y.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    return err


DECODE = [  # (B, H, Tk, D): cfg1 rows, cfg3 / cfg4 rows (few, long: key splits)
    (64, 4, 144, 16),
    (8, 8, 1536, 64),
    (4, 8, 3680, 128),
    (3, 2, 97, 32),
    (2, 3, 33, 10),
    (2, 3, 600, 10),   # key splits with D below its power of two: 2-element slices
    (3, 2, 700, 48),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", DECODE, ids=lambda s: "x".join(map(str, s)))
def test_decode_attention_parity(dev, dtype, shape):
    B, H, Tk, D = shape
    err = _attention_case(dev, dtype, B, H, 1, Tk, D, cache_layout=True, seed=Tk + D)
    assert err <= TOL[dtype], err


PREFILL = [  # (B, H, Tq, Tk, D)
    (2, 4, 96, 96, 16),   # cfg0/1 prefill
    (2, 8, 256, 256, 64),
    (1, 8, 300, 300, 128),
    (2, 3, 5, 17, 32),    # chunked: bottom-right mask (mha.py:69-81)
    (1, 2, 1, 1, 16),     # first token with a cache: Tq == Tk == 1
    (2, 2, 200, 330, 64), # chunked, MFMA path, ragged tiles
    (1, 3, 77, 77, 128),  # Tq not a multiple of the 128-query block
    (1, 2, 640, 640, 64), # several query blocks per head, causal skipping
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", PREFILL, ids=lambda s: "x".join(map(str, s)))
def test_prefill_attention_parity(dev, dtype, shape):
    B, H, Tq, Tk, D = shape
    err = _attention_case(dev, dtype, B, H, Tq, Tk, D, cache_layout=(Tq != Tk), seed=Tq + D)
    assert err <= TOL[dtype], err


def _random_prefills(seed, n):
    """Seeded (B, H, Tq, Tk, D) for the MFMA prefill kernels: D 64 or 128,
    causal (Tq = Tk) or chunked (Tq < Tk), Tq >= 16, ragged query blocks and
    key tiles."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([64, 128]))
        B, H = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        Tk = int(rng.integers(16, 900))
        Tq = Tk if rng.random() < 0.5 else int(rng.integers(16, Tk + 1))
        out.append((B, H, Tq, Tk, D))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_prefills(2024, 12), ids=lambda s: "x".join(map(str, s)))
def test_prefill_attention_random_shapes(dev, dtype, shape):
    """dg_attention at seeded random prefill shapes (the fp32 and the bf16 /
    fp16 MFMA kernels), k and v as strided views of a cache page, against
    float64 attention: fp32 within 1e-5, bf16 / fp16 within 2e-2."""
    B, H, Tq, Tk, D = shape
    err = _attention_case(dev, dtype, B, H, Tq, Tk, D, cache_layout=True, seed=Tq * 7 + Tk + D)
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("amp", [3.0, 20.0])
@pytest.mark.parametrize("shape", [(2, 3, 300, 300, 64), (1, 2, 200, 700, 128)], ids=lambda s: "x".join(map(str, s)))
def test_prefill_attention_large_scores(dev, dtype, amp, shape):
    """Unnormalised q and k scaled by `amp`: scores spread over tens (amp 3)
    or thousands (amp 20) of units, so the MFMA prefill kernels' running
    maximum is raised many times along a row.  Against float64 attention:
    bf16 within 2e-2; fp32 within 1e-5 at amp 3.  At amp 20 a score carries
    fp32 rounding of order 0.1 (64 products of size ~1e5), which moves the
    probabilities of near-tied keys by percents in any fp32 evaluation: there
    the bar is 1.5x the deviation of the reference's own fp32 evaluation (torch
    SDPA on the CPU) from float64, and both are printed."""
    from diff_gpt import _native
    from oracle import torch_ref as tr

    B, H, Tq, Tk, D = shape
    q = _randn((B, Tq, H, D), 7 + D, dtype, amp)
    k = _randn((B, Tk, H, D), 8 + D, dtype, amp)
    v = _randn((B, Tk, H, D), 9 + D, dtype)
    ref = on.attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy())
    y = _native.ops().attention(q.to(dev), k.to(dev), v.to(dev), 1.0 / np.sqrt(D))
    got = y.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    bar = TOL[dtype]
    if dtype == "f32" and amp > 3.0:
        with torch.no_grad():
            own = tr.sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
        own_err = np.abs(own.double().numpy() - ref).max() / np.abs(ref).max()
        print(f"{shape} amp {amp}: ours {err:.3g}, reference fp32 {own_err:.3g} (x max|ref|)", flush=True)
        bar = max(bar, 1.5 * own_err)
    assert err <= bar, (err, bar)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(64, 4, 1, 144, 16), (4, 8, 1, 3000, 64), (2, 2, 1, 5000, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_decode_attention_large_scores(dev, dtype, shape):
    """Single-token decode (the vector kernel, with key splits merged in the
    workgroup or through the workspace) on unnormalised q and k scaled by 3:
    the wave-shared exponent offset is raised several times along the keys;
    fp32 within 1e-5, bf16 within 2e-2 of float64."""
    from diff_gpt import _native

    B, H, Tq, Tk, D = shape
    q = _randn((B, Tq, H, D), 17 + D, dtype, 3.0)
    k = _randn((B, Tk, H, D), 18 + D, dtype, 3.0)
    v = _randn((B, Tk, H, D), 19 + D, dtype)
    ref = on.attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy())
    y = _native.ops().attention(q.to(dev), k.to(dev), v.to(dev), 1.0 / np.sqrt(D))
    got = y.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= TOL[dtype], err


PREFILL_ROPE = [  # (B, H, Tq, Tk, D)
    (2, 3, 200, 200, 64),   # causal, ragged last query block
    (1, 2, 130, 330, 128),  # chunked (bottom-right mask), D = 128
    (2, 2, 16, 16, 64),     # smallest prefill the fused kernel takes
    (1, 2, 640, 640, 128),  # several query blocks per head
]


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("fdt", ["f32", "data"])
@pytest.mark.parametrize("qknorm", [True, False], ids=["qknorm", "rope"])
@pytest.mark.parametrize("shape", PREFILL_ROPE, ids=lambda s: "x".join(map(str, s)))
def test_prefill_rope_equals_rope_then_attention(dev, dtype, fdt, qknorm, shape):
    """dg_prefill_rope rotates (and normalises) q as it loads it; y must be
    bit-identical to dg_rope_qknorm_append on q followed by dg_attention.  q is
    a column slice of a wider projection row (strided), as in the model."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, Tq, Tk, D = shape
    wide = _randn((B, Tq, 3 * H * D), 50 + D, dtype, 2.0).to(dev)
    q = wide[..., H * D : 2 * H * D].view(B, Tq, H, D)
    k = _randn((B, Tk, H, D), 51 + D, dtype).to(dev)
    v = _randn((B, Tk, H, D), 52 + D, dtype).to(dev)
    table = precompute_freqs_cis(D, 2 * Tk, 10000).to(dev)
    freqs = table[Tk - Tq : Tk].view(1, Tq, 1, D // 2, 2)
    if fdt == "data":
        freqs = freqs.to(TDT[dtype])
    scale = 1.0 / D**0.5
    y = torch.empty((B, Tq, H, D), dtype=TDT[dtype], device=dev)
    assert _native.prefill_rope_(q, freqs, k, v, y, scale, qknorm)
    q_rot = torch.empty_like(y)
    _native.rope_qknorm_append_(q, None, None, freqs, q_rot, None, None, qknorm)
    y2 = torch.empty_like(y)
    _native.attention_(q_rot, k, v, y2, scale)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


def _random_rope_prefills(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([64, 128]))
        B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        Tk = int(rng.integers(16, 700))
        Tq = Tk if rng.random() < 0.5 else int(rng.integers(16, Tk + 1))
        out.append((B, H, Tq, Tk, D))
    return out


@pytest.mark.parametrize("qknorm", [True, False])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", _random_rope_prefills(77, 10), ids=lambda s: "x".join(map(str, s)))
def test_prefill_rope_random_shapes(dev, dtype, qknorm, shape):
    """Seeded random causal (Tq = Tk) and chunked (Tq < Tk) shapes: the fused
    RoPE prefill stays bit-identical to RoPE followed by dg_attention."""
    test_prefill_rope_equals_rope_then_attention(dev, dtype, "f32", qknorm, shape)


BOUNDED = [  # (B, H, Tq, Tk, D)
    (2, 3, 200, 200, 64),   # causal, ragged last query block
    (1, 2, 130, 330, 128),  # chunked (bottom-right mask), D = 128
    (2, 2, 16, 16, 64),     # smallest prefill the fused kernel takes
    (1, 2, 640, 640, 128),  # several query blocks per head
    (1, 1, 100, 1000, 64),  # chunk far down a long cache
] + _random_rope_prefills(78, 6)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("fdt", ["f32", "data"])
@pytest.mark.parametrize("shape", BOUNDED, ids=lambda s: "x".join(map(str, s)))
def test_prefill_rope_bounded_against_f64(dev, dtype, fdt, shape):
    """dg_prefill_rope with DG_QKNORM | DG_KEYS_NORMED (keys normalised by
    dg_rope_qknorm_append, as the model's cache holds them): the softmax runs
    without a running maximum on scores in log2 units.  y is within the
    2e-2 * max|ref| bar of float64 attention on the oracle's rotated,
    normalised q and k, and within the same bar of the running-maximum form."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, Tq, Tk, D = shape
    wide = _randn((B, Tq, 3 * H * D), 90 + D, dtype, 2.0).to(dev)
    q = wide[..., H * D : 2 * H * D].view(B, Tq, H, D)
    k = _randn((B, Tk, H, D), 91 + D, dtype, 3.0).to(dev)
    v = _randn((B, Tk, H, D), 92 + D, dtype).to(dev)
    table = precompute_freqs_cis(D, 2 * Tk, 10000)
    kf = table[:Tk].view(1, Tk, 1, D // 2, 2).to(dev)
    qf = table[Tk - Tq : Tk].view(1, Tq, 1, D // 2, 2).to(dev)
    if fdt == "data":
        kf, qf = kf.to(TDT[dtype]), qf.to(TDT[dtype])
    k_rot = torch.empty_like(k)
    _native.rope_qknorm_append_(None, k, None, kf, None, k_rot, None, True)
    scale = 1.0 / D**0.5
    y = torch.empty((B, Tq, H, D), dtype=TDT[dtype], device=dev)
    assert _native.prefill_rope_(q, qf, k_rot, v, y, scale, True, keys_normed=True)
    y_max = torch.empty_like(y)
    assert _native.prefill_rope_(q, qf, k_rot, v, y_max, scale, True)
    torch.cuda.synchronize()
    exp_q = on.rope_qknorm(q.float().cpu().numpy(), qf.float().cpu().numpy(), dtype)
    exp_k = on.rope_qknorm(k.float().cpu().numpy(), kf.float().cpu().numpy(), dtype)
    assert np.array_equal(_bits(k_rot), exp_k.view(np.uint32))
    ref = on.attention_f64(exp_q, exp_k, v.float().cpu().numpy())
    got = y.float().cpu().numpy()
    assert np.abs(got - ref).max() / np.abs(ref).max() <= TOL[dtype]
    two = y_max.float().cpu().numpy()
    assert np.abs(got - two).max() / np.abs(two).max() <= TOL[dtype]


@pytest.mark.parametrize("D", [64, 128])
def test_prefill_rope_keys_normed_large_scale_keeps_running_max(dev, D):
    """DG_KEYS_NORMED with scale = 1: a score reaches +-1.44 * D in log2 units,
    beyond what exp2 keeps inside fp32 (query 0's only visible key is minus
    its own normalised row, query 5 sees its own row as key 5), so the library
    runs the running-maximum form instead: y finite and bit for bit
    dg_attention's on the rotated, normalised q."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, T = 1, 2, 200
    q = _randn((B, T, H, D), 95 + D, "bf16", 2.0)
    k = _randn((B, T, H, D), 96 + D, "bf16")
    k[:, 0] = -q[:, 0]
    k[:, 5] = q[:, 5]
    q, k = q.to(dev), k.to(dev)
    v = _randn((B, T, H, D), 97 + D, "bf16").to(dev)
    freqs = precompute_freqs_cis(D, 2 * T, 10000)[:T].view(1, T, 1, D // 2, 2).to(dev)
    k_rot = torch.empty_like(k)
    _native.rope_qknorm_append_(None, k, None, freqs, None, k_rot, None, True)
    y = torch.empty_like(q)
    assert _native.prefill_rope_(q, freqs, k_rot, v, y, 1.0, True, keys_normed=True)
    q_rot = torch.empty_like(q)
    _native.rope_qknorm_append_(q, None, None, freqs, q_rot, None, None, True)
    y2 = torch.empty_like(q)
    _native.attention_(q_rot, k_rot, v, y2, 1.0)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y.float()).all())
    assert torch.equal(y, y2)
    assert torch.equal(y[:, 0], v[:, 0])  # one visible key: its value


@pytest.mark.parametrize("shape,dtype", [((1, 2, 40, 40, 32), "bf16"), ((1, 2, 40, 40, 32), "f32"),
                                         ((1, 2, 8, 8, 64), "bf16"), ((1, 2, 8, 8, 128), "f32")])
def test_prefill_rope_unsupported_shapes_do_nothing(dev, shape, dtype):
    """Shapes the MFMA kernel does not take return False and leave y alone."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, Tq, Tk, D = shape
    q, k, v = (_randn((B, Tq, H, D), 60 + i, dtype).to(dev) for i in range(3))
    freqs = precompute_freqs_cis(D, 2 * Tk, 10000).to(dev)[:Tq].view(1, Tq, 1, D // 2, 2)
    y = torch.full((B, Tq, H, D), 7.0, dtype=TDT[dtype], device=dev)
    assert not _native.prefill_rope_(q, freqs, k, v, y, 1.0 / D**0.5, True)
    assert bool((y == 7.0).all())


@pytest.mark.parametrize("Tk", [2048, 4096])
def test_decode_split_paths_agree_with_f64(dev, Tk):
    """Key splits of one (row, head) merge inside its workgroup up to 16 of
    them, with no workspace (B*H = 32 at Tk = 2048: 16 splits); more go
    through the workspace and the combine kernel (Tk = 4096: 32 splits) or,
    given no workspace, drop to 16 merged in the workgroup.  Every path
    agrees with fp64."""
    from diff_gpt import _native

    B, H, D = 4, 8, 64
    q = _randn((B, 1, H, D), 1, "bf16").to(dev)
    k = _randn((B, Tk, H, D), 2, "bf16").to(dev)
    v = _randn((B, Tk, H, D), 3, "bf16").to(dev)
    lib = _native.lib()
    assert (lib.dg_attention_workspace_size(B, H, 1, Tk, D, 1) > 0) == (Tk == 4096)
    y_ws = _native.ops().attention(q, k, v, 0.125)  # with the workspace the library asks for
    y_null = torch.empty_like(q)
    st = [ctypes.pointer(_native._bthd_strides(t)) for t in (q, k, v, y_null)]
    rc = lib.dg_attention(B, H, 1, Tk, D, 1, ctypes.c_void_p(q.data_ptr()), st[0],
                          ctypes.c_void_p(k.data_ptr()), st[1], ctypes.c_void_p(v.data_ptr()), st[2],
                          ctypes.c_void_p(y_null.data_ptr()), st[3], 0.125, None, 0,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    if Tk == 2048:
        assert torch.equal(y_ws, y_null)  # one path: no workspace involved
    ref = on.attention_f64(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), 0.125)
    for y in (y_ws, y_null):
        err = np.abs(y.float().cpu().numpy() - ref).max() / np.abs(ref).max()
        assert err <= 2e-2


GROUPED = [  # (B, group, H, prefix, Tk, D)
    (10, 4, 2, 33, 70, 16),
    (12, 6, 8, 600, 1100, 64),
    (4, 2, 8, 1500, 2600, 128),
    (6, 3, 2, 200, 900, 300),   # pair slices: prefix and own keys read pair by pair
    (4, 2, 2, 100, 300, 512),
]
# Groups of >= 16 rows with head_dim 16 / 32 take the matrix-core kernel
# (dg_attn_shared.hip) whenever the vector kernel would not split the keys
# (Tk < 256, or B*H >= 4096): cfg1 (series of 100 rows), a ragged last group,
# a prefix not a multiple of 16 or spanning several 64-key chunks, one own
# key, many own keys, no own key at all.
GROUPED_MFMA = [
    (300, 100, 4, 96, 144, 16),
    (250, 100, 4, 96, 97, 16),
    (70, 16, 2, 33, 70, 32),
    (45, 20, 3, 150, 151, 16),
    (40, 40, 2, 5, 250, 16),
    (32, 16, 2, 50, 50, 32),
    (17, 17, 1, 200, 250, 32),
    (1100, 100, 8, 64, 260, 16),  # B*H >= 4096: no key splits at Tk >= 256 either
    (520, 100, 8, 64, 300, 16),   # B*H = 4160, just past the split threshold
]


def _grouped_case(dtype, shape):
    B, G, H, P, Tk, D = shape
    cap = Tk + 3
    groups = (B + G - 1) // G
    pre = _randn((groups, 2, H, P, D), 70 + D, dtype)
    own = _randn((B, 2, H, Tk - P, D), 71 + D, dtype)
    cache = torch.empty((2, B, H, cap, D), dtype=TDT[dtype])
    cache[:, :, :, :P] = pre.repeat_interleave(G, dim=0)[:B].transpose(0, 1)
    cache[:, :, :, P:Tk] = own.transpose(0, 1)
    q = _randn((B, 1, H, D), 72 + D, dtype)
    return q, cache


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", GROUPED, ids=lambda s: "x".join(map(str, s)))
def test_grouped_prefix_attention_equals_plain(dev, dtype, shape):
    """Rows of a group share their first `prefix` cache positions (a broadcast
    prefill, kv_cache.py:77-79): reading the prefix from the group's first row
    gives the very bits of the plain decode, and both match fp64."""
    from diff_gpt import _native

    B, G, H, P, Tk, D = shape
    q, cache = _grouped_case(dtype, shape)
    cd, qd = cache.to(dev), q.to(dev)
    keys = cd[0, :, :, :Tk].transpose(1, 2)
    vals = cd[1, :, :, :Tk].transpose(1, 2)
    ops = _native.ops()
    y_plain = ops.attention(qd, keys, vals, 1.0 / np.sqrt(D))
    y_grp = ops.attention(qd, keys, vals, 1.0 / np.sqrt(D), P, G)
    assert torch.equal(y_grp, y_plain)
    ref = on.attention_f64(q.float().numpy(), keys.float().cpu().numpy(), vals.float().cpu().numpy())
    err = np.abs(y_grp.float().cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", GROUPED_MFMA, ids=lambda s: "x".join(map(str, s)))
def test_grouped_prefix_attention_mfma(dev, dtype, shape):
    """The shared prefix on MFMA, own keys on the VALU: against fp64 at the
    north-star bars, against the plain decode kernel within them, and the
    device-position entry point (graph form) bit-identical to the eager call
    at the same position."""
    from diff_gpt import _native

    B, G, H, P, Tk, D = shape
    q, cache = _grouped_case(dtype, shape)
    cd, qd = cache.to(dev), q.to(dev)
    keys = cd[0, :, :, :Tk].transpose(1, 2)
    vals = cd[1, :, :, :Tk].transpose(1, 2)
    ops = _native.ops()
    y_plain = ops.attention(qd, keys, vals, 1.0 / np.sqrt(D))
    y_grp = ops.attention(qd, keys, vals, 1.0 / np.sqrt(D), P, G)
    ref = on.attention_f64(q.float().numpy(), keys.float().cpu().numpy(), vals.float().cpu().numpy())
    scale = np.abs(ref).max()
    err = np.abs(y_grp.float().cpu().numpy() - ref).max() / scale
    assert err <= TOL[dtype], err
    gap = (y_grp.float() - y_plain.float()).abs().max().item() / scale
    assert gap <= TOL[dtype], gap
    # graph form: positions 0 .. pos of the full-capacity cache views
    y_at = torch.empty_like(qd)
    pos = torch.tensor([Tk - 1], dtype=torch.int32, device=dev)
    _native.decode_attention_at_(qd, cd[0].transpose(1, 2), cd[1].transpose(1, 2), y_at, 1.0 / np.sqrt(D),
                                 pos, P, G)
    assert torch.equal(y_at, y_grp)


def _decode_splits(BH: int, keys: int) -> int:
    """The host's key-split count for a decode launch over ``keys`` keys
    (restated to tell which launches should agree bit for bit): enough splits
    to give 4096 waves, at least 128 keys each, at most 64."""
    return max(1, min(-(-4096 // BH), keys // 128, 64))


DECODE_STEP = [  # (B, group, H, prefix, pos, D, cap)
    (300, 100, 4, 96, 120, 16, 144),  # cfg1 series: one launch
    (70, 16, 2, 33, 69, 32, 80),      # D = 32, prefix not a multiple of 16
    (45, 20, 3, 150, 150, 16, 160),   # no cached own key: the new one only
    # own-key register sets of 4 (fp32) / 8 (16-bit) keys at D = 16: one set,
    # two sets, and a refill round then two sets (fp32) / two sets (16-bit)
    (40, 20, 2, 64, 66, 16, 80),
    (40, 20, 2, 64, 71, 16, 80),
    (40, 20, 2, 64, 79, 16, 96),
    # pos + 1 below the 256 keys at which decode splits the keys, capacity
    # above: both position forms choose the kernel and its splits for the
    # capacity, so they still agree bit for bit (ragged last group)
    (155, 100, 2, 188, 243, 32, 261),
    (200, 100, 2, 188, 243, 16, 261),
    (6, 1, 4, 0, 23, 16, 40),         # no shared prefix: the vector kernel's fused step
    # no shared prefix, pos + 1 = 201 keys (one split) but max_pos = 300 (two):
    # y is dg_decode_attention_at's over max_pos, not the two calls' bits
    (1, 1, 1, 0, 200, 16, 300),
    (12, 6, 8, 600, 700, 64, 720),    # small groups, D = 64 (key splits): the vector kernel's fused step
    (1, 1, 2, 0, 4000, 64, 4100),     # 32 key splits: the fused step's partials through the workspace
    # head dims past 128: vector slices (512), pair slices (300, 1000),
    # a shared prefix at D = 384, the workspace at D = 1000
    (2, 1, 2, 0, 300, 512, 320),
    (3, 1, 2, 0, 100, 300, 130),
    (4, 2, 2, 50, 120, 384, 140),
    (4, 2, 2, 50, 120, 300, 140),
    (1, 1, 2, 0, 3000, 1000, 3100),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", DECODE_STEP, ids=lambda s: "x".join(map(str, s)))
def test_decode_step_matches_two_calls(dev, dtype, shape):
    """dg_decode_step == dg_rope_qknorm_append at pos + dg_attention_grouped over
    0 .. pos: the cache bit for bit.  Where the attention runs on the vector
    kernel (its fused one-launch step), y bit for bit dg_decode_attention_at's
    over max_pos = cap (kernel and key splits chosen for the capacity), and
    the two calls' wherever those choose the same number of key splits;
    within the north-star bars of them and of fp64 where the shared-prefix
    kernel fuses the step or the split counts differ.  The device-position
    form equal to the host-position form; an out-of-range device position
    leaves the cache untouched."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, G, H, P, pos, D, cap = shape
    groups = (B + G - 1) // G
    cache = torch.zeros((2, B, H, cap, D), dtype=TDT[dtype])
    if P:
        pre = _randn((groups, 2, H, P, D), 80 + D, dtype)
        cache[:, :, :, :P] = pre.repeat_interleave(G, dim=0)[:B].transpose(0, 1)
    cache[:, :, :, P:pos] = _randn((B, 2, H, pos - P, D), 81 + D, dtype).transpose(0, 1)
    q, k, v = (_randn((B, 1, H, D), 82 + D + i, dtype, 2.0).to(dev) for i in range(3))
    table = precompute_freqs_cis(D, 2 * cap, 10000).to(TDT[dtype]).to(dev)
    scale = 1.0 / np.sqrt(D)
    prefix, group = (P, G) if G > 1 else (0, 1)
    ops = _native.ops()

    c1 = cache.to(dev)
    q_rot = torch.empty_like(q)
    ops.rope_qknorm_append(q, k, v, table[pos:pos + 1].view(1, 1, 1, D // 2, 2), q_rot,
                           c1[0, :, :, pos:pos + 1].transpose(1, 2), c1[1, :, :, pos:pos + 1].transpose(1, 2), True)
    keys, vals = c1[0, :, :, :pos + 1].transpose(1, 2), c1[1, :, :, :pos + 1].transpose(1, 2)
    y1 = ops.attention(q_rot, keys, vals, scale, prefix, group)

    c2, y2 = cache.to(dev), torch.empty_like(q)
    _native.decode_step_(q, k, v, table[pos], c2[0].transpose(1, 2), c2[1].transpose(1, 2), y2, scale, pos,
                         prefix, group)
    assert torch.equal(c2, c1)
    same_splits = _decode_splits(B * H, pos + 1) == _decode_splits(B * H, cap)
    fused = G >= 16 and D in (16, 32) and _decode_splits(B * H, cap) == 1
    if fused or not same_splits:
        ref = on.attention_f64(q_rot.float().cpu().numpy(), keys.float().cpu().numpy(), vals.float().cpu().numpy(),
                               scale)
        mag = np.abs(ref).max()
        assert np.abs(y2.float().cpu().numpy() - ref).max() <= TOL[dtype] * mag
        assert (y2.float() - y1.float()).abs().max().item() <= TOL[dtype] * mag
    if not fused:
        y_at = torch.empty_like(q)
        _native.decode_attention_at_(q_rot, c1[0].transpose(1, 2), c1[1].transpose(1, 2), y_at, scale,
                                     torch.tensor([pos], dtype=torch.int32, device=dev), prefix, group)
        assert torch.equal(y2, y_at)
        if same_splits:
            assert torch.equal(y2, y1)

    c3, y3 = cache.to(dev), torch.empty_like(q)
    p = torch.tensor([pos], dtype=torch.int32, device=dev)
    _native.decode_step_(q, k, v, table, c3[0].transpose(1, 2), c3[1].transpose(1, 2), y3, scale, p, prefix, group)
    assert torch.equal(c3, c2) and torch.equal(y3, y2)

    c4 = cache.to(dev)
    _native.decode_step_(q, k, v, table, c4[0].transpose(1, 2), c4[1].transpose(1, 2), torch.empty_like(q), scale,
                         torch.tensor([cap], dtype=torch.int32, device=dev), prefix, group)
    torch.cuda.synchronize()
    assert torch.equal(c4.cpu(), cache)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(6, 1, 4, 0, 23, 16, 40), (3, 1, 2, 0, 70, 64, 100), (2, 1, 2, 0, 600, 128, 700),
                                   (2, 1, 2, 0, 300, 512, 320), (1, 1, 1, 0, 900, 1000, 1000)],
                         ids=lambda s: "x".join(map(str, s)))
def test_decode_step_ignores_old_contents_at_the_position(dev, dtype, shape):
    """The fused decode step appends the new key and value while it streams
    the keys: the cache rows at and past the position hold NaN before the
    step (stale or uninitialised memory), yet y equals the two calls' (which
    append first) bit for bit, with the host and the device position, and the
    cache holds the new row."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, G, H, P, pos, D, cap = shape
    cache = torch.full((2, B, H, cap, D), float("nan"), dtype=TDT[dtype])
    cache[:, :, :, :pos] = _randn((B, 2, H, pos, D), 91 + D, dtype).transpose(0, 1)
    q, k, v = (_randn((B, 1, H, D), 92 + D + i, dtype, 2.0).to(dev) for i in range(3))
    table = precompute_freqs_cis(D, 2 * cap, 10000).to(TDT[dtype]).to(dev)
    scale = 1.0 / np.sqrt(D)
    ops = _native.ops()
    c1 = cache.to(dev)
    q_rot = torch.empty_like(q)
    ops.rope_qknorm_append(q, k, v, table[pos:pos + 1].view(1, 1, 1, D // 2, 2), q_rot,
                           c1[0, :, :, pos:pos + 1].transpose(1, 2), c1[1, :, :, pos:pos + 1].transpose(1, 2), True)
    y_at = torch.empty_like(q)
    _native.decode_attention_at_(q_rot, c1[0].transpose(1, 2), c1[1].transpose(1, 2), y_at, scale,
                                 torch.tensor([pos], dtype=torch.int32, device=dev))
    for p_arg in (pos, torch.tensor([pos], dtype=torch.int32, device=dev)):
        c2, y2 = cache.to(dev), torch.empty_like(q)
        _native.decode_step_(q, k, v, table if isinstance(p_arg, torch.Tensor) else table[pos],
                             c2[0].transpose(1, 2), c2[1].transpose(1, 2), y2, scale, p_arg)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(y2).all())
        assert torch.equal(y2, y_at)
        assert torch.equal(c2[:, :, :, :pos + 1], c1[:, :, :, :pos + 1])


def _random_decode_steps(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([16, 32]))
        G = int(rng.choice([1, 16, 17, 50, 100, 128]))
        B = int(rng.integers(1, 3 * G + 1)) if G > 1 else int(rng.integers(1, 64))  # ragged last group
        H = int(rng.integers(1, 5))
        P = int(rng.integers(0, 200)) if G > 1 else 0
        pos = P + int(rng.integers(0, 80))  # pos == P: no cached own key
        cap = pos + 1 + int(rng.integers(0, 40))  # pos + 1 and cap either side of 256 at times
        out.append((B, G, H, P, pos, D, cap))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_decode_steps(4242, 16), ids=lambda s: "x".join(map(str, s)))
def test_decode_step_random_shapes(dev, dtype, shape):
    """Seeded random (rows, group, heads, prefix, position, head_dim, capacity)
    through the same checks as the fixed decode-step cases."""
    test_decode_step_matches_two_calls(dev, dtype, shape)


# ------------------------------------------------------------------ wide and odd head dims

# Every even head_dim up to 1024 runs on the RoPE and vector attention
# kernels.  A row padded to the next power of two spreads over at most 64
# lanes: vector slices of max(16 bytes, DPAD / 64) elements where D is a
# multiple of them and the operands are aligned to a load (96, 192, 384, 512,
# 1024 here), else pair slices read pair by pair with the pairs past D skipped
# (130, 300 and 1000 here; any D past 128 whose operands are aligned to a
# pair only).
WIDE_D = [96, 130, 192, 300, 384, 512, 1000, 1024]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", WIDE_D)
def test_rope_qknorm_append_wide_head_dims(dev, dtype, D):
    """RoPE + QK-norm + append at head dims past 128: q and k bit-exact
    against the oracle (the norm's pairwise tree over the padded row is the
    same whatever the slice width), v copied, the rest of the cache
    untouched."""
    _rope_append_case(dev, dtype, 2, 5, 3, D, 7, 16)


def _misaligned(t: torch.Tensor) -> torch.Tensor:
    """t's values in a view one pair into rows of D + 2 elements: aligned to
    a pair, not to a 16-byte load, row strides not multiples of 4."""
    buf = torch.zeros((*t.shape[:-1], t.shape[-1] + 2), dtype=t.dtype, device=t.device)
    view = buf[..., 2:]
    view.copy_(t)
    return view


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("D", [256, 512, 1024])
def test_rope_pair_slices_on_misaligned_rows(dev, dtype, D):
    """q, k and v as views aligned to a pair only: the kernel reads and
    writes its slices pair by pair, with the vector path's bits."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, T, H, pos, cap = 2, 4, 3, 5, 12
    q = _randn((B, T, H, D), 11 + D, dtype, 2.0)
    k = _randn((B, T, H, D), 21 + D, dtype, 2.0)
    v = _randn((B, T, H, D), 31 + D, dtype)
    fc = precompute_freqs_cis(D, 64, 10000).to(TDT[dtype])[pos:pos + T].view(1, T, 1, D // 2, 2)
    qd, kd, vd = (_misaligned(t.to(dev)) for t in (q, k, v))
    cd = torch.zeros((2, B, H, cap, D), dtype=TDT[dtype], device=dev)
    q_out = _misaligned(torch.zeros_like(q).to(dev))
    _native.ops().rope_qknorm_append(qd, kd, vd, fc.to(dev), q_out, cd[0, :, :, pos:pos + T].transpose(1, 2),
                                     cd[1, :, :, pos:pos + T].transpose(1, 2), True)
    torch.cuda.synchronize()
    fcn = fc.float().numpy()
    got = cd.cpu()
    assert np.array_equal(_bits(q_out), on.rope_qknorm(q.float().numpy(), fcn, dtype).view(np.uint32))
    assert np.array_equal(_bits(got[0, :, :, pos:pos + T].transpose(1, 2)),
                          on.rope_qknorm(k.float().numpy(), fcn, dtype).view(np.uint32))
    assert torch.equal(got[1, :, :, pos:pos + T].transpose(1, 2), v)
    assert (got[:, :, :, :pos] == 0).all() and (got[:, :, :, pos + T:] == 0).all()


WIDE_ATTN = [  # (B, H, Tq, Tk, D)
    (2, 2, 1, 700, 512),    # decode, key splits merged in the workgroup
    (1, 2, 1, 5000, 1024),  # decode, 39 key splits: workspace and combine (8 merge in a workgroup at 1024)
    (3, 2, 1, 300, 1000),   # pair slices
    (2, 2, 1, 1200, 300),   # pair slices with key splits
    (2, 2, 1, 500, 130),    # pair slices of 4 elements
    (2, 2, 1, 500, 192),    # vector slices, D below its power of two
    (1, 2, 70, 70, 384),    # causal prefill
    (1, 1, 33, 50, 1000),   # chunked prefill, pair slices
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", WIDE_ATTN, ids=lambda s: "x".join(map(str, s)))
def test_attention_wide_head_dims(dev, dtype, shape):
    """dg_attention at head dims past 128 against float64 at the north-star
    bars."""
    B, H, Tq, Tk, D = shape
    err = _attention_case(dev, dtype, B, H, Tq, Tk, D, cache_layout=(Tq != Tk), seed=Tk + D)
    assert err <= TOL[dtype], err


def _random_wide(seed, n):
    """Seeded (B, H, Tq, Tk, D, misaligned): any even D from 2 to 1024,
    decode, causal or chunked, the operands aligned to a pair only in about
    a third of the cases."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = 2 * int(rng.integers(1, 513))
        Tk = int(rng.integers(1, 1000))
        Tq = min(int(rng.choice([1, Tk, int(rng.integers(1, Tk + 1))])), 400)
        Tk = max(Tk, Tq)
        out.append((int(rng.integers(1, 4)), int(rng.integers(1, 4)), Tq, Tk, D, bool(rng.random() < 0.35)))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_wide(31, 14), ids=lambda s: "x".join(map(str, s)))
def test_rope_and_attention_random_head_dims(dev, dtype, shape):
    """Seeded random even head dims up to 1024, aligned or aligned to a pair
    only: RoPE + QK-norm bit-exact against the oracle, then attention over
    the rotated rows within the north-star bars of float64."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, Tq, Tk, D, mis = shape
    seed = D + Tk
    q = _randn((B, Tq, H, D), seed, dtype, 2.0)
    k = _randn((B, Tk, H, D), seed + 1, dtype, 2.0)
    v = _randn((B, Tk, H, D), seed + 2, dtype)
    fq = precompute_freqs_cis(D, 2 * Tk, 10000).to(TDT[dtype])
    fq_q = fq[Tk - Tq:Tk].view(1, Tq, 1, D // 2, 2)
    fq_k = fq[:Tk].view(1, Tk, 1, D // 2, 2)
    put = _misaligned if mis else (lambda t: t)
    qd, kd, vd = (put(t.to(dev)) for t in (q, k, v))
    q_rot = put(torch.zeros_like(q).to(dev))
    k_rot = put(torch.zeros_like(k).to(dev))
    v_out = put(torch.zeros_like(v).to(dev))
    ops = _native.ops()
    ops.rope_qknorm_append(qd, None, None, fq_q.to(dev), q_rot, None, None, True)
    ops.rope_qknorm_append(None, kd, vd, fq_k.to(dev), None, k_rot, v_out, True)
    exp_q = on.rope_qknorm(q.float().numpy(), fq_q.float().numpy(), dtype)
    exp_k = on.rope_qknorm(k.float().numpy(), fq_k.float().numpy(), dtype)
    assert np.array_equal(_bits(q_rot), exp_q.view(np.uint32))
    assert np.array_equal(_bits(k_rot), exp_k.view(np.uint32))
    assert torch.equal(v_out.cpu(), v)
    y = put(torch.zeros_like(q).to(dev))
    _native.attention_(q_rot, k_rot, v_out, y, 1.0 / np.sqrt(D))
    ref = on.attention_f64(exp_q.astype(np.float64), exp_k.astype(np.float64), v.float().numpy().astype(np.float64))
    assert np.abs(y.float().cpu().numpy() - ref).max() <= TOL[dtype] * np.abs(ref).max()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 2, 1, 600, 512), (1, 2, 40, 40, 256), (1, 1, 1, 3000, 1024)],
                         ids=lambda s: "x".join(map(str, s)))
def test_attention_pair_slices_on_misaligned_rows(dev, dtype, shape):
    """q, k, v and y aligned to a pair only (power-of-two head dims that
    would take vector slices): pair slices, within the bars of float64."""
    from diff_gpt import _native

    B, H, Tq, Tk, D = shape
    q = _randn((B, Tq, H, D), 5 + D, dtype)
    k = _randn((B, Tk, H, D), 6 + D, dtype)
    v = _randn((B, Tk, H, D), 7 + D, dtype)
    ref = on.attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy())
    qd, kd, vd = (_misaligned(t.to(dev)) for t in (q, k, v))
    y = _misaligned(torch.zeros_like(q).to(dev))
    _native.attention_(qd, kd, vd, y, 1.0 / np.sqrt(D))
    got = y.float().cpu().numpy().astype(np.float64)
    assert np.abs(got - ref).max() <= TOL[dtype] * np.abs(ref).max()


# ------------------------------------------------------------------ strided copy


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_copy4d_exact_with_broadcast(dev, dtype):
    from diff_gpt import _native

    src = _randn((1, 3, 5, 7), 9, dtype).to(dev)
    dst = torch.zeros((4, 3, 5, 7), dtype=TDT[dtype], device=dev)
    _native.ops().copy4d(src.expand(4, 3, 5, 7), dst)
    assert torch.equal(dst.cpu(), src.cpu().expand(4, 3, 5, 7))
    # transposed destination view
    dst2 = torch.zeros((3, 4, 7, 5), dtype=TDT[dtype], device=dev)
    _native.ops().copy4d(src.expand(4, 3, 5, 7).transpose(0, 1).transpose(2, 3), dst2)
    assert torch.equal(dst2.cpu(), src.cpu().expand(4, 3, 5, 7).transpose(0, 1).transpose(2, 3))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_copy4d_row_vector_path(dev, dtype):
    """Rows with a contiguous, 16-byte-multiple last dimension take the
    row-vectorised kernel: batch broadcast of a cache prefix into strided
    pages (KVCache.prefill), exact."""
    from diff_gpt import _native

    L2, B, H, T, D, cap = 4, 6, 3, 10, 16, 13
    src = _randn((L2, 1, H, cap * D), 11, dtype).to(dev)
    big = torch.full((L2, B, H, cap * D), -1.0, dtype=TDT[dtype], device=dev)
    dst = big[..., : T * D]
    _native.ops().copy4d(src[..., : T * D].expand(L2, B, H, T * D), dst)
    ref = torch.full((L2, B, H, cap * D), -1.0, dtype=TDT[dtype])
    ref[..., : T * D] = src[..., : T * D].cpu().expand(L2, B, H, T * D)
    assert torch.equal(big.cpu(), ref)


def _random_copies(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        shape = tuple(int(x) for x in rng.integers(1, 9, size=3)) + (int(rng.choice([1, 3, 8, 16, 24, 64, 200])),)
        bcast = tuple(bool(b) for b in rng.random(4) < 0.3)  # broadcast (stride 0) source dims
        perm = tuple(int(x) for x in rng.permutation(4))    # destination storage order
        out.append((shape, bcast, perm))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("case", _random_copies(5, 12), ids=lambda c: "x".join(map(str, c[0])) + "-" + "".join(
    "b" if b else "." for b in c[1]) + "-" + "".join(map(str, c[2])))
def test_copy4d_random_strides(dev, dtype, case):
    """Seeded random shapes, broadcast source dims and destination layouts
    (a permuted storage order, then a slice of a wider buffer): exact, and
    nothing outside the destination view is written."""
    from diff_gpt import _native

    shape, bcast, perm = case
    src_shape = tuple(1 if b else n for n, b in zip(shape, bcast))
    src = _randn(src_shape, sum(shape) + 7 * sum(bcast), dtype).to(dev).expand(shape)
    store = [shape[i] for i in perm]
    store[-1] += 5  # wider rows: the view's last storage dimension is a slice
    buf = torch.full(store, -3.0, dtype=TDT[dtype], device=dev)
    view = buf[..., : shape[perm[-1]]]
    inv = [perm.index(i) for i in range(4)]
    dst = view.permute(*inv)
    assert dst.shape == shape
    _native.ops().copy4d(src, dst)
    assert torch.equal(dst.cpu(), src.cpu())
    assert bool((buf[..., shape[perm[-1]]:] == -3.0).all())


# ------------------------------------------------------------------ seeded random shapes


def _random_shapes(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([16, 32, 64, 128, 48, 10]))
        kind = rng.choice(["decode", "prefill", "chunk"])
        B, H = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        if kind == "decode":
            Tq, Tk = 1, int(rng.integers(1, 1200))
        elif kind == "prefill":
            Tq = Tk = int(rng.integers(2, 400))
        else:
            Tk = int(rng.integers(3, 500))
            Tq = int(rng.integers(2, Tk))
        out.append((B, H, Tq, Tk, D))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_shapes(2024, 16), ids=lambda s: "x".join(map(str, s)))
def test_attention_random_shapes(dev, dtype, shape):
    """dg_attention on seeded random (B, H, Tq, Tk, D): decode, causal prefill
    and chunked prefill, every kernel family, against fp64 brute force."""
    B, H, Tq, Tk, D = shape
    err = _attention_case(dev, dtype, B, H, Tq, Tk, D, cache_layout=(Tq != Tk), seed=B * 131 + Tq + Tk + D)
    assert err <= TOL[dtype], err


def _random_groups(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        G = int(rng.choice([16, 20, 37, 64, 100]))
        B = int(rng.integers(G, 3 * G + 1))
        P = int(rng.integers(1, 200))
        Tk = P + int(rng.integers(0, 60))
        out.append((B, G, int(rng.integers(1, 5)), P, max(Tk, 1), int(rng.choice([16, 32]))))
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", _random_groups(7, 10), ids=lambda s: "x".join(map(str, s)))
def test_grouped_prefix_random_shapes(dev, dtype, shape):
    """The two-wave shared-prefix kernel on seeded random groups (ragged
    groups, prefixes not multiples of 16, zero to 59 own keys) against fp64."""
    from diff_gpt import _native

    B, G, H, P, Tk, D = shape
    q, cache = _grouped_case(dtype, shape)
    cd, qd = cache.to(dev), q.to(dev)
    keys = cd[0, :, :, :Tk].transpose(1, 2)
    vals = cd[1, :, :, :Tk].transpose(1, 2)
    y = _native.ops().attention(qd, keys, vals, 1.0 / np.sqrt(D), P, G)
    ref = on.attention_f64(q.float().numpy(), keys.float().cpu().numpy(), vals.float().cpu().numpy())
    err = np.abs(y.float().cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= TOL[dtype], err


# ------------------------------------------------------------------ shared prefix stored once

PREFIX_PAGES = [  # (B, group, H, P, pos, D, dtype)
    (32, 16, 4, 96, 120, 16, "f32"),    # shared kernel (MFMA prefix), configs[1] geometry
    (48, 16, 2, 40, 40, 32, "bf16"),    # shared kernel, first decode step (no own key yet)
    (8, 4, 2, 50, 70, 64, "bf16"),      # vector kernel with a prefix
    (3, 1, 2, 40, 45, 32, "f32"),       # one row per group: each row's own prefix page
    (4, 2, 8, 2000, 2100, 128, "bf16"), # vector kernel with key splits
]


def _split_case(dev, B, group, H, P, pos, D, dtype, seed):
    """A broadcast cache (every row of a group holds its group's prefix) and
    the same contents as prefix pages + own pages (positions P.. only)."""
    cap = pos + 8
    G = B // group
    dense = _randn((2, B, H, cap, D), seed, dtype).to(dev)
    dense.view(2, G, group, H, cap, D)[..., :P, :] = dense.view(2, G, group, H, cap, D)[:, :, :1, :, :P, :]
    pages = dense.view(2, G, group, H, cap, D)[:, :, 0, :, :P, :].contiguous()  # (2, G, H, P, D)
    own = dense[..., P:, :].contiguous()  # (2, B, H, cap - P, D)
    return dense, pages, own


@pytest.mark.parametrize("shape", PREFIX_PAGES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("device_pos", [False, True], ids=["host_pos", "device_pos"])
def test_decode_step_prefix_pages_equal_broadcast_rows(dev, shape, device_pos):
    """dg_decode_step with the prefix in pages of its own (dg_prefix k/v,
    own_start = P) computes and writes exactly what it does on the broadcast
    cache that holds the prefix in every row: same y bits, same appended
    key/value, nothing written below own_start."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, group, H, P, pos, D, dtype = shape
    dense, pages, own = _split_case(dev, B, group, H, P, pos, D, dtype, 7 + D)
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(B, 1, H, D, generator=g).to(TDT[dtype]).to(dev) for _ in range(3))
    table = precompute_freqs_cis(D, 2 * (pos + 8), 10000).to(dev).to(TDT[dtype])
    if device_pos:
        p, freqs = torch.tensor([pos], dtype=torch.int32, device=dev), table
    else:
        p, freqs = pos, table[pos]
    scale = D ** -0.5
    y0 = torch.empty_like(q)
    _native.decode_step_(q, k, v, freqs, dense[0].transpose(1, 2), dense[1].transpose(1, 2), y0, scale, p, P, group)
    y1 = torch.empty_like(q)
    pre = _native.Prefix(P, group, pages[0].transpose(1, 2), pages[1].transpose(1, 2), P)
    pages_before = pages.clone()
    _native.decode_step_(q, k, v, freqs, own[0].transpose(1, 2), own[1].transpose(1, 2), y1, scale, p, prefix=pre)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    assert torch.equal(own, dense[..., P:, :])
    assert torch.equal(pages, pages_before)


@pytest.mark.parametrize("shape", PREFIX_PAGES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("Tq", [1, 5])
def test_attention_prefix_pages_equal_broadcast_rows(dev, shape, Tq):
    """dg_attention_grouped over prefix pages + own pages: the decode (Tq = 1)
    and a 5-query chunk give the bits of the broadcast cache."""
    from diff_gpt import _native

    B, group, H, P, pos, D, dtype = shape
    dense, pages, own = _split_case(dev, B, group, H, P, pos, D, dtype, 11 + D)
    Tk = pos + 1
    q = _randn((B, Tq, H, D), 12, dtype).to(dev)
    scale = D ** -0.5
    y0 = torch.empty_like(q)
    _native.attention_(q, dense[0, :, :, :Tk].transpose(1, 2), dense[1, :, :, :Tk].transpose(1, 2), y0, scale,
                       P, group)
    y1 = torch.empty_like(q)
    pre = _native.Prefix(P, group, pages[0].transpose(1, 2), pages[1].transpose(1, 2), P)
    _native.attention_(q, own[0, :, :, :Tk - P].transpose(1, 2), own[1, :, :, :Tk - P].transpose(1, 2), y1, scale,
                       prefix=pre)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
