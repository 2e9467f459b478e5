"""Decode attention at the BASELINE.json configurations' own decode geometry,
and the attention inside the bf16 configs[3] / configs[4] models isolated at
the north-star bar.

Kernel instances (the host's split rule: key splits only when B*H falls short
of 4096 waves and a split keeps at least 128 keys; up to 16 splits are the
waves of one workgroup and merge in LDS):
  * configs[3] decode, B=512 H=8 D=64, L_kv 1025 .. 1536: B*H = 4096 units, no
    split -- attn_vec_kernel<T, 64, 8, 2, false>, one wave per (row, head)
    walking all its keys;
  * configs[4] decode, B=64 H=8 D=128, L_kv 3585 .. 3680: 512 units x 8 key
    splits merged in the workgroup -- attn_vec_kernel<T, 128, 8, 2, true>;
  * B=8 H=8 D=128, L_kv 1500: 64 units x 11 splits merged in the workgroup
    (a split count that is not a power of two, in fp32 at 1e-5 as well).

Every output row is compared with float64 attention computed on the device
(torch, float64 elementwise products and sums) over the same q, K and V; the first, middle
and last unit and a few seeded ones are compared with the CPU oracle
(oracle.numerics.attention_head_f64) as well.  Bars: fp32 1e-5, bf16 / fp16
2e-2, each relative to the unit's own max|ref|.  Some units carry a planted
dominant key at a split boundary (the last key of one split and the first of
the next), so that the largest score of the row sits where two splits meet.

The decode step (dg_decode_step, device position as the captured model runs
it, max_pos = capacity) at the same shapes: the appended key bit-exact against
the oracle's RoPE + QK-norm, the value copied, nothing else in the cache
written, and y against float64 attention on the oracle's rotated query.
"""

import numpy as np
import pytest
import torch

from oracle import numerics as on

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 1e-5, "bf16": 2e-2, "f16": 2e-2}


def _splits(BH: int, keys: int) -> int:
    """The host's key-split count for a decode launch (restated to name the
    kernel instance each case runs): enough splits to give 4096 waves, at
    least 128 keys each, at most 64."""
    want = -(-4096 // BH)
    return max(1, min(want, keys // 128, 64))


DECODE_GEOMETRY = [  # (B, H, D, Tk, dtype)
    (512, 8, 64, 1025, "bf16"),   # configs[3], first decode step
    (512, 8, 64, 1536, "bf16"),   # configs[3], last decode step
    (512, 8, 64, 1536, "f32"),
    (64, 8, 128, 3585, "bf16"),   # configs[4], first decode step
    (64, 8, 128, 3680, "bf16"),   # configs[4], last decode step
    (64, 8, 128, 3680, "f32"),
    (64, 8, 128, 3585, "f16"),
    (8, 8, 128, 1500, "f32"),     # 11 splits merged in the workgroup
    (8, 8, 128, 1500, "f16"),
    (8, 8, 128, 1500, "bf16"),
]


def _ids(s):
    return "x".join(map(str, s))


def _device_randn(shape, seed, dev, dtype, scale=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * scale).to(TDT[dtype])


def _sampled_units(BH: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    return sorted({0, BH // 2, BH - 1, *(int(u) for u in rng.integers(0, BH, 4))})


def _plant_boundary_keys(q, kc, Tk, units, nsplit):
    """Plant a large score at key j*split_len - 1 (the last of split j - 1) of
    some sampled units and at key j*split_len (the first of split j) of
    others: k <- c * q there, with c = 3 (score 3*|q|^2*scale: the key takes
    nearly all the weight) or c = 1/4 (about a fifth of it, the rest spread
    over every split)."""
    B, _, H, D = q.shape
    if nsplit == 1:
        bounds = [Tk // 2 - 1, Tk // 2, Tk - 1]
    else:
        split_len = ((-(-Tk // nsplit)) + 15) // 16 * 16
        bounds = [split_len * j + d for j in range(1, nsplit) for d in (-1, 0) if split_len * j < Tk]
    for n, u in enumerate(units[1:]):  # unit 0 keeps plain random keys
        b, h = divmod(u, H)
        c = 3.0 if n % 2 == 0 else 0.25
        kc[b, h, bounds[(n // 2) % len(bounds)]] = (c * q[b, 0, h].float()).to(kc.dtype)


def _f64_rows(q, kc, vc, Tk, scale, chunk=256):
    """float64 attention of every (row, head) on the device, by elementwise
    products and sums (no library GEMM): q (B,1,H,D), kc / vc (B,H,cap,D) ->
    (B*H, D) float64."""
    B, _, H, D = q.shape
    qq = q[:, 0].to(torch.float64).reshape(B * H, D)
    out = torch.empty((B * H, D), dtype=torch.float64, device=q.device)
    kf, vf = kc.reshape(B * H, kc.size(2), D), vc.reshape(B * H, vc.size(2), D)
    for u0 in range(0, B * H, chunk):
        u1 = min(B * H, u0 + chunk)
        kk = kf[u0:u1, :Tk].to(torch.float64)
        s = (kk * qq[u0:u1, None, :]).sum(-1) * scale  # (n, Tk)
        del kk
        s = s - s.amax(dim=-1, keepdim=True)
        p = torch.exp(s)
        p = p / p.sum(dim=-1, keepdim=True)
        vv = vf[u0:u1, :Tk].to(torch.float64)
        out[u0:u1] = (p[..., None] * vv).sum(1)
    return out


def _check_rows(y, ref64, units_cpu, tol, what):
    """y (B,1,H,D) against the float64 rows: every unit on the device, per-unit
    relative to its own max|ref|; ``units_cpu`` maps sampled units to the CPU
    oracle's rows."""
    B, _, H, D = y.shape
    got = y[:, 0].reshape(B * H, D).to(torch.float64)
    mag = ref64.abs().amax(dim=1).clamp_min(1e-30)
    rel = ((got - ref64).abs().amax(dim=1) / mag)
    worst = int(rel.argmax())
    assert float(rel[worst]) <= tol, (what, "unit", worst, float(rel[worst]))
    for u, ref in units_cpu.items():
        g = got[u].cpu().numpy()
        err = np.abs(g - ref).max() / np.abs(ref).max()
        assert err <= tol, (what, "unit", u, err)
    return float(rel.max())


@pytest.mark.parametrize("shape", DECODE_GEOMETRY, ids=_ids)
def test_decode_attention_at_config_geometry(dev, shape):
    from diff_gpt import _native

    B, H, D, Tk, dtype = shape
    ns = _splits(B * H, Tk)
    print(f"decode geometry B={B} H={H} D={D} Tk={Tk} {dtype}: {ns} key split(s)", flush=True)
    cap = Tk + 7
    seed = Tk + D + B
    q = _device_randn((B, 1, H, D), seed, dev, dtype, 2.0)
    kc = _device_randn((B, H, cap, D), seed + 1, dev, dtype)
    vc = _device_randn((B, H, cap, D), seed + 2, dev, dtype)
    units = _sampled_units(B * H, seed)
    _plant_boundary_keys(q, kc, Tk, units, ns)
    scale = 1.0 / np.sqrt(D)
    ws = _native.lib().dg_attention_workspace_size(B, H, 1, Tk, D, _native._dtype_code(q))
    assert (ws == 0) == (ns <= 16), (ns, ws)  # merged in the workgroup: no workspace
    y = torch.empty_like(q)
    keys, vals = kc[:, :, :Tk].transpose(1, 2), vc[:, :, :Tk].transpose(1, 2)
    _native.attention_(q, keys, vals, y, scale)
    ref64 = _f64_rows(q, kc, vc, Tk, scale)
    cpu = {}
    for u in units:
        b, h = divmod(u, H)
        cpu[u] = on.attention_head_f64(q[b, :, h].float().cpu().numpy(), kc[b, h, :Tk].float().cpu().numpy(),
                                       vc[b, h, :Tk].float().cpu().numpy(), scale)[0]
        # the device float64 reference agrees with the CPU oracle (far inside
        # the tightest bar, fp32's 1e-5)
        assert np.abs(ref64[u].cpu().numpy() - cpu[u]).max() <= 1e-7 * np.abs(cpu[u]).max()
    worst = _check_rows(y, ref64, cpu, TOL[dtype], "dg_attention")
    print(f"  worst per-unit error {worst:.3g} (bar {TOL[dtype]})", flush=True)


@pytest.mark.parametrize("shape", DECODE_GEOMETRY, ids=_ids)
def test_decode_step_at_config_geometry(dev, shape):
    """dg_decode_step with the position on the device at pos = Tk - 1 (the
    step's key is the last of Tk), capacity Tk + 9: the graph-captured form
    the model runs, choosing its kernel and splits for the capacity."""
    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, D, Tk, dtype = shape
    pos, cap = Tk - 1, Tk + 9
    print(f"decode step geometry B={B} H={H} D={D} pos={pos} cap={cap} {dtype}: "
          f"{_splits(B * H, cap)} key split(s)", flush=True)
    seed = 7 * Tk + D + B
    cache = _device_randn((2, B, H, cap, D), seed, dev, dtype)
    before = cache.clone()
    q, k, v = (_device_randn((B, 1, H, D), seed + 1 + i, dev, dtype, 2.0) for i in range(3))
    table = precompute_freqs_cis(D, 2 * cap, 10000).to(TDT[dtype])
    scale = 1.0 / np.sqrt(D)
    y = torch.empty_like(q)
    p = torch.tensor([pos], dtype=torch.int32, device=dev)
    _native.decode_step_(q, k, v, table.to(dev), cache[0].transpose(1, 2), cache[1].transpose(1, 2), y, scale, p)
    torch.cuda.synchronize()

    cs = table[pos].float().numpy()
    exp_q = on.rope_qknorm(q.float().cpu().numpy(), cs, dtype)  # (B, 1, H, D)
    exp_k = on.rope_qknorm(k.float().cpu().numpy(), cs, dtype)
    got_k = cache[0, :, :, pos].float().cpu().numpy()  # (B, H, D)
    assert np.array_equal(got_k.view(np.uint32), exp_k[:, 0].view(np.uint32))
    assert torch.equal(cache[1, :, :, pos], v[:, 0])
    # nothing but position pos written
    assert torch.equal(cache[..., :pos, :], before[..., :pos, :])
    assert torch.equal(cache[..., pos + 1:, :], before[..., pos + 1:, :])

    q_rot = torch.from_numpy(exp_q).to(TDT[dtype]).to(dev)
    ref64 = _f64_rows(q_rot, cache[0], cache[1], pos + 1, scale)
    cpu = {}
    for u in _sampled_units(B * H, seed):
        b, h = divmod(u, H)
        cpu[u] = on.attention_head_f64(exp_q[b, :, h].astype(np.float64), cache[0, b, h, :pos + 1].float().cpu().numpy(),
                                       cache[1, b, h, :pos + 1].float().cpu().numpy(), scale)[0]
    worst = _check_rows(y, ref64, cpu, TOL[dtype], "dg_decode_step")
    print(f"  worst per-unit error {worst:.3g} (bar {TOL[dtype]})", flush=True)


# ------------------------------------------------------------------ attention inside the bf16 models


class _AttentionTap:
    """Records, for chosen layers, what the HIP path feeds the attention and
    what it returns: the layer's q/k/v/g projections (the argument of the
    attention module's _attend, which Block.forward calls on them), and the
    arguments and output of the prefill (dg_prefill_rope) and decode-step
    (dg_decode_step) calls made while that layer attends."""

    def __init__(self, model, layers, monkeypatch):
        from diff_gpt import _native

        self.records = {l: [] for l in layers}
        self._cur = None
        for l in layers:
            sa = model.blocks[l].sa
            monkeypatch.setattr(sa, "_attend", self._wrap(l, sa._attend))
        orig_prefill, orig_step = _native.prefill_rope_, _native.decode_step_

        def prefill(q, freqs, k, v, y, scale, qknorm, keys_normed=False):
            ok = orig_prefill(q, freqs, k, v, y, scale, qknorm, keys_normed)
            if self._cur is not None:
                self._cur.update(kind="prefill", q=q.clone(), freqs=freqs.clone(), keys=k.clone(), values=v.clone(),
                                 y=y.clone(), scale=scale, fused=ok, keys_normed=keys_normed)
            return ok

        def step(q, k, v, freqs, k_cache, v_cache, y, scale, pos, *args, **kw):
            orig_step(q, k, v, freqs, k_cache, v_cache, y, scale, pos, *args, **kw)
            if self._cur is not None:
                self._cur.update(kind="step", q=q.clone(), k=k.clone(), v=v.clone(), freqs=freqs.clone(),
                                 y=y.clone(), scale=scale, pos=pos)

        monkeypatch.setattr(_native, "prefill_rope_", prefill)
        monkeypatch.setattr(_native, "decode_step_", step)

    def _wrap(self, layer, attend):
        def wrapped(qkvg, freqs_cis, kv_cache):
            self._cur = {"qkvg": qkvg.detach().clone()}
            self.records[layer].append(self._cur)
            try:
                return attend(qkvg, freqs_cis, kv_cache)
            finally:
                self._cur = None
        return wrapped

    def close(self):
        pass


def _projections(model, layer, qkvg):
    """q, k, v (B,T,H,D): the column slices of the layer's projections."""
    sa = model.blocks[layer].sa
    H, D = sa.n_head, sa.head_dim
    inner = H * D
    B, T, _ = qkvg.shape
    return tuple(qkvg[..., i * inner:(i + 1) * inner].reshape(B, T, H, D) for i in range(3))


def _check_layer_attention(model, layer, recs, D, what):
    """The recorded prefill and first decode step of one layer against float64
    attention over the oracle's rotated and normalised q and k (from the same
    projections), per (row, head) at 2e-2 * max|ref|; the cache keys the HIP
    path attended over equal the oracle's bit for bit."""
    pre, step = recs[0], recs[1]
    assert pre["kind"] == "prefill" and pre["fused"] and pre["keys_normed"], what
    assert step["kind"] == "step", what
    q, k, v = _projections(model, layer, pre["qkvg"])
    assert torch.equal(q, pre["q"]), what  # the projections the kernel was fed
    B, T, H, _ = q.shape
    cs = pre["freqs"].float().cpu().numpy().reshape(T, D // 2, 2)
    exp_q = on.rope_qknorm(q.float().cpu().numpy(), cs[None, :, None], "bf16")
    exp_k = on.rope_qknorm(k.float().cpu().numpy(), cs[None, :, None], "bf16")
    assert np.array_equal(pre["keys"].float().cpu().numpy().view(np.uint32), exp_k.view(np.uint32)), what
    vn = v.float().cpu().numpy()
    y = pre["y"].float().cpu().numpy()
    worst = 0.0
    for b in range(B):
        for h in range(H):
            ref = on.attention_head_f64(exp_q[b, :, h], exp_k[b, :, h], vn[b, :, h], pre["scale"])
            err = np.abs(y[b, :, h] - ref).max() / np.abs(ref).max()
            worst = max(worst, err)
            assert err <= 2e-2, (what, "prefill", b, h, err)
    # decode step at position T: keys 0 .. T-1 from the prefill, key T new
    qs, ks, vs = _projections(model, layer, step["qkvg"])
    assert torch.equal(qs, step["q"]) and torch.equal(ks, step["k"]), what
    cs1 = step["freqs"].float().cpu().numpy().reshape(1, D // 2, 2)
    sq = on.rope_qknorm(qs.float().cpu().numpy(), cs1[None, :, None], "bf16")
    sk = on.rope_qknorm(ks.float().cpu().numpy(), cs1[None, :, None], "bf16")
    ys = step["y"].float().cpu().numpy()
    for b in range(B):
        for h in range(H):
            keys = np.concatenate([exp_k[b, :, h], sk[b, :, h]])
            vals = np.concatenate([vn[b, :, h], vs[b, :, h].float().cpu().numpy()])
            ref = on.attention_head_f64(sq[b, :, h], keys, vals, step["scale"])
            err = np.abs(ys[b, :, h] - ref).max() / np.abs(ref).max()
            worst = max(worst, err)
            assert err <= 2e-2, (what, "decode", b, h, err)
    return worst


@pytest.mark.parametrize("geom", ["cfg3", "cfg4"])
def test_attention_inside_bf16_config_models(dev, geom, monkeypatch):
    """The bf16 configs[3] model (n_embd 512, 8 heads of 64, 8 layers) at
    B = 2 with a 1024-token prompt, and the configs[4] model (n_embd 1024, 8
    heads of 128, 4 layers) at B = 1 with a 3584-token prompt: a prefill and
    one decode step over the KV cache.  For the first and the last layer, the
    attention output the model computed (dg_prefill_rope with the bounded
    softmax, then dg_decode_step) is within 2e-2 * max|ref| of float64
    attention over the oracle's RoPE + QK-norm of the very projections the
    layer produced, for every (row, head) and every query row."""
    from diff_gpt.model.gpt import GPT
    from diff_gpt.model.kv_cache import KVCache

    n_embd, n_head, n_layer, B, T = (512, 8, 8, 2, 1024) if geom == "cfg3" else (1024, 8, 4, 1, 3584)
    D = n_embd // n_head
    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=n_embd, block_size=2048, n_head=n_head, n_layer=n_layer,
                use_checkpoint=False).eval().to(torch.bfloat16).to(dev)
    layers = [0, n_layer - 1]
    tap = _AttentionTap(model, layers, monkeypatch)
    prompts = torch.randint(0, 256, (B, T), generator=torch.Generator().manual_seed(3))
    kv = KVCache(batch_size=B, num_heads=n_head, seq_len=T + 1, head_dim=D, num_layers=n_layer)
    with torch.inference_mode():
        logits = model(prompts.to(dev), kv_cache=kv)[0][:, -1]
        model(logits.argmax(-1, keepdim=True), kv_cache=kv)
    torch.cuda.synchronize()
    tap.close()
    for l in layers:
        worst = _check_layer_attention(model, l, tap.records[l], D, f"{geom} layer {l}")
        print(f"{geom} bf16 model, layer {l}: attention worst error {worst:.3g} x max|ref| (bar 2e-2)", flush=True)
