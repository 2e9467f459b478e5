"""Benchmark of diff-gpt's attention hot path on one MI355X.

Default workload: 64 series x 100 trajectories =
6400 concurrent sequences of the README GPT geometry (2 layers, 4 heads,
head_dim 16), a shared 96-token prefix per series already broadcast into the
KV cache, then 48 decode steps (L_kv 97..144).  One bench step = that whole
decode job through the hot path: per decode step and layer, one
dg_decode_step launch (RoPE + QK-norm + KV append + decode attention) on
synthetic q/k/v projections resident in HBM.

    python bench.py [--steps K] [--warmup W] [--dtype fp32|bf16] [--no-prefill]
                    [--no-shapes | --shapes-only] [--no-cpu-baseline] [--traffic-json FILE]

Prints ONE JSON line.  value = sequences*48*K / timed seconds (tokens/s); the
job's 96 launches are captured once in a HIP graph (as Engine captures its
decode step) and the K timed steps are K graph replays.  roofline = the
decode-step kernel: algorithmic bytes per launch over its mean launch time,
timed with HIP events on the launch stream around K replays of the graph (so
the graph's short gaps between kernels count as kernel time).  Bytes per
(row, head): es*(2*L_kv*D + 4*D) -- K+V of every visible position, q, y, the
k/v projections read and appended; in shared mode the prefix rows count once
per series.  The decode_unfused leg runs the same job as two launches per
layer-step (RoPE/append, then attention) and reports the attention kernel
alone (es*(2*L_kv*D + 2*D) per (row, head)).  The prefill leg (configs[2]:
B=256, H=8, T=1024, D=64, bf16, RoPE + QK-norm, causal) reports TFLOP/s of
the model's prefill kernel with FLOP = 2*B*H*D*T*(T+1).  The shapes leg times
decode and prefill attention alone at configs[3] / configs[4] shapes; the
jobs leg runs configs[3]'s and configs[4]'s whole decode jobs through the
captured decode step, and both configurations end to end through
Engine.generate_multi_batch; the engine leg runs configs[1] end to end as one
call and as the reference's 64 per-series calls.  cpu_baseline = the
oracle's torch-CPU restatement of the reference decode path on sampled steps
of the job (warm-up, median of 5), on this host's cores; the prefill and
engine legs carry baselines of their own.
"""

from __future__ import annotations

import argparse
import ctypes
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (REPO / "diff-gpt_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_MFMA_PEAK_TFLOPS = 157.3
METRIC = "decode attn tokens/s + % HBM roofline; prefill attn TFLOP/s, 1×MI355X"

# configs[1] geometry
SERIES, TRAJ, PREFIX, NEW = 64, 100, 96, 48
LAYERS, HEADS, HEAD_DIM = 2, 4, 16


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def decode_job(dtype_name: str, steps: int, warmup: int, shared: bool = False, fused: bool = True):
    import torch

    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    dev = torch.device("cuda:0")
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    es = 4 if dt == torch.float32 else 2
    ops = _native.ops()
    B, H, D, L = SERIES * TRAJ, HEADS, HEAD_DIM, LAYERS
    cap = PREFIX + NEW
    g = torch.Generator(device=dev).manual_seed(0)

    # shared: the KVCache.prefill layout -- each series' 96-token prefix once,
    # as (L,2,SERIES,H,PREFIX,D) pages, and each row's pages holding positions
    # PREFIX.. only; plain: every row's (L,2,B,H,cap,D) pages hold the whole
    # prefix (the reference's broadcast copy) and are read as such
    prefix = torch.randn((L, 2, SERIES, H, PREFIX, D), generator=g, device=dev).to(dt)
    if shared:
        own0 = PREFIX
        cache = torch.empty((L, 2, B, H, NEW, D), dtype=dt, device=dev)
    else:
        own0 = 0
        cache = torch.empty((L, 2, B, H, cap, D), dtype=dt, device=dev)
        cache.view(L, 2, SERIES, TRAJ, H, cap, D)[..., :PREFIX, :] = prefix.unsqueeze(3)
    table = precompute_freqs_cis(D, 2 * 138, 10000).to(dev).to(dt)
    # synthetic projections for every (step, layer): q, k, v (B,1,H,D)
    qkv = torch.randn((NEW, L, 3, B, 1, H, D), generator=g, device=dev).to(dt)
    q_rot = torch.empty((B, 1, H, D), dtype=dt, device=dev)
    y = torch.empty((B, 1, H, D), dtype=dt, device=dev)
    torch.cuda.synchronize()

    # The job calls the C-ABI directly with argument packs prepared once, on a
    # stream of its own, and is captured in a HIP graph, as the Engine's decode
    # step is: the 192 launches of a job then run back to back with no host
    # in between.
    lib = _native.lib()
    side = torch.cuda.Stream()
    stream = ctypes.c_void_p(side.cuda_stream)
    code = _native._DTYPE_CODE[dt]
    P = ctypes.pointer
    S3 = _native._bthd_strides
    packs = []
    keep = []  # ctypes objects the argument packs point at
    if shared:
        pre_arg = [None] * L
        for layer in range(L):
            pk, pv = prefix[layer, 0].transpose(1, 2), prefix[layer, 1].transpose(1, 2)
            pre_arg[layer], _ = _native._prefix_arg(_native.Prefix(PREFIX, TRAJ, pk, pv, PREFIX))
        keep.append(pre_arg)
    else:
        pre_arg = [None] * L
    for s in range(NEW):
        t0 = PREFIX + s
        fc = table[t0:t0 + 1].view(1, 1, 1, D // 2, 2)
        for layer in range(L):
            q, k, v = qkv[s, layer]
            if fused:
                # one launch: RoPE + QK-norm + append at t0 + attention over 0..t0
                kc = cache[layer, 0].transpose(1, 2)
                vc = cache[layer, 1].transpose(1, 2)
                assert lib.dg_decode_step_workspace_size(B, H, cap, D, code) == 0
                args = (B, H, D, code, _native._ptr(q), P(S3(q)), _native._ptr(k), P(S3(k)),
                        _native._ptr(v), P(S3(v)), _native._ptr(kc), P(S3(kc)), _native._ptr(vc), P(S3(vc)),
                        _native._ptr(table[t0]), 0, code, t0, None, cap, _native._ptr(y), P(S3(y)),
                        0.25, pre_arg[layer], _native.DG_QKNORM, None, 0, stream)
                packs.append((None, args))
                continue
            kd = cache[layer, 0, :, :, t0 - own0:t0 - own0 + 1].transpose(1, 2)
            vd = cache[layer, 1, :, :, t0 - own0:t0 - own0 + 1].transpose(1, 2)
            keys = cache[layer, 0, :, :, :t0 + 1 - own0].transpose(1, 2)
            vals = cache[layer, 1, :, :, :t0 + 1 - own0].transpose(1, 2)
            rope_args = (B, 1, H, D, code,
                         _native._ptr(q), P(S3(q)), _native._ptr(q_rot), P(S3(q_rot)),
                         _native._ptr(k), P(S3(k)), _native._ptr(kd), P(S3(kd)),
                         _native._ptr(v), P(S3(v)), _native._ptr(vd), P(S3(vd)),
                         _native._ptr(fc), P(_native.Stride3(0, 0, 0)), code, _native.DG_QKNORM, stream)
            ws = lib.dg_attention_workspace_size(B, H, 1, t0 + 1, D, code)
            assert ws == 0, "configs[1] decode runs without key splits"
            attn_args = (B, H, 1, t0 + 1, D, code,
                         _native._ptr(q_rot), P(S3(q_rot)), _native._ptr(keys), P(S3(keys)),
                         _native._ptr(vals), P(S3(vals)), _native._ptr(y), P(S3(y)),
                         0.25, pre_arg[layer], None, 0, stream)
            packs.append((rope_args, attn_args))
    rope_fn = lib.dg_rope_qknorm_append
    attn_fn = lib.dg_decode_step if fused else lib.dg_attention_grouped

    def run(with_rope: bool, upto: int | None = None):
        for rope_args, attn_args in packs[:upto]:
            if with_rope and rope_args is not None and rope_fn(*rope_args) != 0:
                raise RuntimeError(lib.dg_last_error().decode())
            if attn_fn(*attn_args) != 0:
                raise RuntimeError(lib.dg_last_error().decode())

    with torch.cuda.stream(side):
        run(True, upto=1)  # one eager layer-step loads the code objects before capture
    torch.cuda.synchronize()
    job, attn_only = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(job, stream=side):
        run(True)
    with torch.cuda.graph(attn_only, stream=side):
        run(False)
    with torch.cuda.stream(side):
        for _ in range(warmup):  # untimed warm-up jobs: graph replays, as the timed ones
            job.replay()
    torch.cuda.synchronize()
    log(f"decode {dtype_name}: warmup done, timing {steps} jobs")
    with torch.cuda.stream(side):
        t_start = time.perf_counter()
        for _ in range(steps):
            job.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t_start
        # decode-attention launches alone (the same 96 per job), bracketed by
        # events on their stream: mean launch duration including the graph's
        # small gaps between kernels
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(side)
        for _ in range(steps):
            attn_only.replay()
        b.record(side)
        torch.cuda.synchronize()
    launches = steps * len(packs)
    attn_s = a.elapsed_time(b) / 1e3
    mean_kernel_s = attn_s / launches
    # algorithmic bytes per launch, averaged over the job's L_kv = 97..144:
    # K+V rows of every visible position, q, y; the fused step also reads the
    # k, v projections and writes them to the cache (and takes the new
    # position's K+V from registers instead of the cache), + 2*D per (row,
    # head) in all; with a shared prefix the prefix rows count once per series
    # (unique bytes)
    extra = 2 * D if fused else 0
    if shared:
        bytes_job = sum(H * es * (2 * D * (PREFIX * SERIES + (s + 1) * B) + (2 * D + extra) * B)
                        for s in range(NEW)) * L
    else:
        bytes_job = sum(B * H * es * (2 * (PREFIX + s + 1) * D + 2 * D + extra) for s in range(NEW)) * L
    bytes_per_launch = bytes_job / (NEW * L)
    achieved = bytes_per_launch / mean_kernel_s / 1e9
    tokens = B * NEW * steps
    return {
        "tokens_per_s": tokens / elapsed,
        "ms_per_step": elapsed / steps * 1e3,
        "kernel_mean_us": mean_kernel_s * 1e6,
        "bytes_per_launch": bytes_per_launch,
        "achieved_gbs": achieved,
        "launches": launches,
        "attn_only_tokens_per_s": B * NEW * steps / attn_s,
    }


def prefill_leg(reps: int = 10, traffic_json: str | None = None):
    """B=256, T=1024, H=8, D=64 bf16, q/k/v in (B,T,H,D) projection
    layout, RoPE base 1e4 + QK-norm, causal.  The model's prefill step is two
    launches: RoPE + QK-norm of k (dg_rope_qknorm_append), then
    dg_prefill_rope, which rotates and normalises q as it loads it and -- the
    keys being normalised -- runs its softmax without a running maximum.
    fused_ms: that attention kernel alone (the headline TFLOP/s and
    roofline); with_rope_ms: the two-launch step; attn_ms: dg_attention on an
    already rotated q (general kernel, running maximum); with_rope_unfused_ms:
    RoPE on q and k in the first launch, dg_attention in the second.  Each is
    a graph of `reps` back-to-back launches timed with HIP events on its
    stream, median of 3 replays."""
    import torch

    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    dev = torch.device("cuda:0")
    B, T, H, D = 256, 1024, 8, 64
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn((B, T, H, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    fc = precompute_freqs_cis(D, 2 * T, 10000).to(dev).to(torch.bfloat16)[:T].view(1, T, 1, D // 2, 2)
    q_rot, k_rot, y = (torch.empty_like(q) for _ in range(3))
    ops = _native.ops()
    flop = 2.0 * B * H * D * T * (T + 1)
    scale = 1.0 / D**0.5

    def fused_kernel():
        if not _native.prefill_rope_(q, fc, k_rot, v, y, scale, True, keys_normed=True):
            raise RuntimeError("configs[2] prefill is not taken by dg_prefill_rope")

    def model_step():
        ops.rope_qknorm_append(None, k, None, fc, None, k_rot, None, True)
        fused_kernel()

    def unfused_step():
        ops.rope_qknorm_append(q, k, None, fc, q_rot, k_rot, None, True)
        _native.attention_(q_rot, k_rot, v, y, scale)

    def attn_alone():
        _native.attention_(q_rot, k_rot, v, y, scale)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        unfused_step()
        model_step()
    torch.cuda.synchronize()
    legs = {"fused": fused_kernel, "model": model_step, "unfused": unfused_step, "attn": attn_alone}
    graphs = {}
    for name, fn in legs.items():
        graphs[name] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[name], stream=side):
            for _ in range(reps):
                fn()
    times = {name: [] for name in legs}
    with torch.cuda.stream(side):
        for _ in range(3):
            for name, graph in graphs.items():
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(side)
                graph.replay()
                b.record(side)
                torch.cuda.synchronize()
                times[name].append(a.elapsed_time(b) / 1e3 / reps)
    t = {name: sorted(v)[1] for name, v in times.items()}
    tf = flop / t["fused"] / 1e12
    # HBM bytes per attention launch, from the committed rocprofv3 counter runs
    traffic = None
    if traffic_json and Path(traffic_json).exists():
        traffic = json.loads(Path(traffic_json).read_text()).get("prefill_cfg2_bf16")
    return {
        "workload": "configs[2] causal prefill B=256 H=8 T=1024 D=64 bf16, RoPE+QK-norm",
        "tflops": tf,
        "fused_ms": t["fused"] * 1e3,
        "with_rope_ms": t["model"] * 1e3,
        "tflops_with_rope": flop / t["model"] / 1e12,
        "attn_ms": t["attn"] * 1e3,
        "attn_tflops": flop / t["attn"] / 1e12,
        "with_rope_unfused_ms": t["unfused"] * 1e3,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / BF16_PEAK_TFLOPS, "traffic": traffic},
    }


def prefill_cpu_baseline(batch: int = 8, runs: int = 5):
    """configs[2] on the host cores: the reference's prefill attention path
    (rope.py, rms_norm.py at mha.py:48, SDPA with is_causal, mha.py:44-64) in
    torch on the CPU, bf16, at B = `batch` of the 256 sequences; one warm-up,
    then the median of `runs`; TFLOP/s over the same FLOP count, time
    extrapolated linearly to B = 256 (rows are independent)."""
    import torch

    from oracle import torch_ref as tr

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    T, H, D = 1024, 8, 64
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn((batch, T, H, D), generator=g).to(torch.bfloat16) for _ in range(3))
    fc = tr.freqs_table(D, 2 * T, 10000).to(torch.bfloat16)[:T].view(1, T, 1, D // 2, 2)

    def run():
        qq, kk = tr.rms(tr.rope(q, fc)), tr.rms(tr.rope(k, fc))
        return tr.sdpa(qq.transpose(1, 2), kk.transpose(1, 2), v.transpose(1, 2))

    with torch.no_grad():
        run()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            run()
            ts.append(time.perf_counter() - t0)
    med = sorted(ts)[len(ts) // 2]
    flop = 2.0 * batch * H * D * T * (T + 1)
    return {
        "value": flop / med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"configs[2] prefill (RoPE + QK-norm + causal SDPA, bf16) at B={batch} of 256, "
                  f"median of {runs} after a warm-up; {med * 1e3:.1f} ms, extrapolated to "
                  f"{med * 256 / batch * 1e3:.0f} ms for B=256 (linear in B)",
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def shapes_leg(reps: int = 20):
    """Decode and prefill attention alone at the larger configs' shapes, bf16,
    plain per-row caches: configs[3] (B=512, H=8, D=64; decode at L_kv = 1025,
    the first step after the 1024-token prefill, and 1536, the last; prefill
    T=1024) and configs[4] (B=64, H=8, D=128; decode at L_kv = 3585 and 3680;
    prefill T=3584).  The cache is (2, B, H, capacity, D), the layout the
    model's KV cache uses.  Each case is `reps` launches captured in one graph,
    timed with events over 5 replays (median); decode bytes per launch =
    B*H*es*(2*L_kv*D + 2*D), prefill FLOP = 2*B*H*D*T*(T+1).  The same two
    prefills in fp32 (an fp32 model of that geometry) run on the fp32 matrix
    cores and are priced against their 157.3 TFLOP/s peak.  The D = 16 fp32
    prefills of configs[0] (B=32) and configs[1] (one series, B=1), T=96,
    H=4, are launch-bound and report latency only."""
    import torch

    from diff_gpt import _native

    dev = torch.device("cuda:0")
    dt, es = torch.bfloat16, 2

    def timed(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(reps):
                fn()
        ts = []
        with torch.cuda.stream(side):
            for _ in range(5):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(side)
                graph.replay()
                b.record(side)
                torch.cuda.synchronize()
                ts.append(a.elapsed_time(b) / 1e3 / reps)
        return sorted(ts)[2]

    out = []
    g = torch.Generator(device=dev).manual_seed(0)
    for name, B, H, D, cap, lens in (("configs[3]", 512, 8, 64, 1536, (1025, 1536)),
                                     ("configs[4]", 64, 8, 128, 3680, (3585, 3680))):
        cache = torch.randn((2, B, H, cap, D), generator=g, device=dev).to(dt)
        q = torch.randn((B, 1, H, D), generator=g, device=dev).to(dt)
        y = torch.empty_like(q)
        for L in lens:
            keys = cache[0, :, :, :L].transpose(1, 2)
            vals = cache[1, :, :, :L].transpose(1, 2)
            t = timed(lambda: _native.attention_(q, keys, vals, y, D ** -0.5))
            nbytes = B * H * es * (2 * L * D + 2 * D)
            out.append({"workload": f"{name} decode attention B={B} H={H} D={D} L_kv={L} bf16",
                        "us": t * 1e6, "achieved_gbs": nbytes / t / 1e9,
                        "frac": nbytes / t / 1e9 / HBM_PEAK_GBS})
            log(f"shapes: {out[-1]}")
        del cache, q, y
    from diff_gpt.model.rope import precompute_freqs_cis

    for name, B, H, D, T in (("configs[3]", 512, 8, 64, 1024), ("configs[4]", 64, 8, 128, 3584)):
        q, k, v = (torch.randn((B, T, H, D), generator=g, device=dev).to(dt) for _ in range(3))
        fc = precompute_freqs_cis(D, 2 * T, 10000).to(dev).to(dt)[:T].view(1, T, 1, D // 2, 2)
        k_rot = torch.empty_like(k)
        _native.ops().rope_qknorm_append(None, k, None, fc, None, k_rot, None, True)
        y = torch.empty_like(q)
        flop = 2.0 * B * H * D * T * (T + 1)
        # the model's prefill kernel: q rotated and normalised as it is
        # loaded, normalised keys, bounded softmax
        t = timed(lambda: _native.prefill_rope_(q, fc, k_rot, v, y, D ** -0.5, True, keys_normed=True))
        # the general kernel (any q, k: running maximum)
        t_gen = timed(lambda: _native.attention_(q, k, v, y, D ** -0.5))
        tf = flop / t / 1e12
        out.append({"workload": f"{name} causal prefill attention B={B} H={H} T={T} D={D} bf16, "
                                "q RoPE + QK-norm fused, bounded softmax (the model's kernel)",
                    "ms": t * 1e3, "tflops": tf, "frac": tf / BF16_PEAK_TFLOPS,
                    "general_kernel_tflops": flop / t_gen / 1e12})
        log(f"shapes: {out[-1]}")
        del q, k, v, y, k_rot
    # an fp32 model of the same geometry: dg_attention on rotated q and k runs
    # the fp32 MFMA kernel (v_mfma_f32_32x32x2_f32, dense fp32 matrix peak
    # 157.3 TFLOP/s)
    for name, B, H, D, T in (("configs[3]", 512, 8, 64, 1024), ("configs[4]", 64, 8, 128, 3584)):
        q, k, v = (torch.randn((B, T, H, D), generator=g, device=dev) for _ in range(3))
        y = torch.empty_like(q)
        flop = 2.0 * B * H * D * T * (T + 1)
        t = timed(lambda: _native.attention_(q, k, v, y, D ** -0.5))
        tf = flop / t / 1e12
        out.append({"workload": f"{name} geometry causal prefill attention B={B} H={H} T={T} D={D} fp32 "
                                "(an fp32 model's prefill kernel, on the matrix cores)",
                    "ms": t * 1e3, "tflops": tf, "frac": tf / FP32_MFMA_PEAK_TFLOPS,
                    "peak_tflops": FP32_MFMA_PEAK_TFLOPS})
        log(f"shapes: {out[-1]}")
        del q, k, v, y
    # configs[0] and configs[1] prefill (D = 16, fp32): launch-bound, so the
    # figure is latency per launch, with no roofline
    for name, B in (("configs[0]", 32), ("configs[1] per series", 1)):
        H, D, T = 4, 16, 96
        q, k, v = (torch.randn((B, T, H, D), generator=g, device=dev) for _ in range(3))
        y = torch.empty_like(q)
        t = timed(lambda: _native.attention_(q, k, v, y, D ** -0.5))
        out.append({"workload": f"{name} causal prefill attention B={B} H={H} T={T} D={D} fp32",
                    "us": t * 1e6, "bound": "latency"})
        log(f"shapes: {out[-1]}")
        del q, k, v, y
    return out


DECODE_JOBS = {  # name: (rows, heads, head_dim, layers, prompt length, decode steps)
    "configs[3]": (512, 8, 64, 8, 1024, 512),
    "configs[4]": (64, 8, 128, 4, 3584, 96),
}


def decode_job_leg(name: str, reps: int = 2):
    """A whole decode job of configs[3] / configs[4] through the decode-step
    entry point, bf16: the cache (L,2,B,H,capacity,D) holds the prompt's
    keys and values, then every step appends one position per row and
    attends over all of them, layer by layer (dg_decode_step: RoPE + QK-norm
    + append + decode attention with key splits), on synthetic projections
    resident in HBM.  The step is captured once with the position read on the
    device (as the Engine replays it) and replayed for every step of the job.
    Bytes per (row, head, step) = es*(2*L_kv*D + 4*D) (every visible position's
    K and V, q, y, the new k and v read and appended)."""
    import torch

    from diff_gpt import _native
    from diff_gpt.model.rope import precompute_freqs_cis

    B, H, D, L, T0, steps = DECODE_JOBS[name]
    dev = torch.device("cuda:0")
    dt, es = torch.bfloat16, 2
    cap = T0 + steps
    g = torch.Generator(device=dev).manual_seed(0)
    cache = torch.empty((L, 2, B, H, cap, D), dtype=dt, device=dev)
    for layer in range(L):
        cache[layer, :, :, :, :T0] = torch.randn((2, B, H, T0, D), generator=g, device=dev).to(dt)
    proj = torch.randn((L, 3, B, 1, H, D), generator=g, device=dev).to(dt)
    table = precompute_freqs_cis(D, 2 * cap, 10000).to(dev).to(dt)
    pos = torch.full((1,), T0, dtype=torch.int32, device=dev)
    y = torch.empty((B, 1, H, D), dtype=dt, device=dev)

    def step():
        for layer in range(L):
            q, k, v = proj[layer]
            _native.decode_step_(q, k, v, table, cache[layer, 0].transpose(1, 2), cache[layer, 1].transpose(1, 2),
                                 y, D ** -0.5, pos)
        pos.add_(1)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step()
    times = []
    with torch.cuda.stream(side):
        for _ in range(reps):
            pos.fill_(T0)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(side)
            for _ in range(steps):
                graph.replay()
            b.record(side)
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) / 1e3)
    t = min(times)
    nbytes = sum(B * H * es * (2 * (T0 + s + 1) * D + 4 * D) for s in range(steps)) * L
    out = {"workload": f"{name} decode job: B={B} H={H} D={D} {L} layers, {steps} steps, "
                       f"L_kv {T0 + 1}..{cap}, bf16, dg_decode_step per layer-step (captured)",
           "tokens_per_s": B * steps / t, "seconds": t, "bytes": nbytes,
           "achieved_gbs": nbytes / t / 1e9, "frac": nbytes / t / 1e9 / HBM_PEAK_GBS}
    del cache, proj
    return out


def engine_multi_leg(name: str):
    """A configuration end to end through Engine.generate_multi_batch (the
    whole model, prefill included, random-init weights, bf16):
    configs[3] -- 512 prompts of 1024 uniform ids, 512 greedy steps;
    configs[4] -- 64 prompts of 3584 ids (7 channels x 512 steps), 96 steps
    with a schedule per prompt forcing channels 0, 1 and 2 from seeded
    uniform ids, greedy elsewhere.  One warm-up call (captures the decode
    step), then one timed call."""
    import numpy as np
    import torch

    from diff_gpt.model.engine import Engine
    from diff_gpt.model.gpt import GPT
    from diff_gpt.sampler.temperature import TemperatureSampler

    dev = torch.device("cuda:0")
    if name == "configs[3]":
        C, H, L, n, T, steps = 512, 8, 8, 512, 1024, 512
    else:
        C, H, L, n, T, steps = 1024, 8, 4, 64, 3584, 96
    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=C, block_size=2048, n_head=H, n_layer=L,
                use_checkpoint=False).eval().to(dev).to(torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    prompts = torch.randint(0, 256, (n, T), generator=g).tolist()
    sched = None
    if name == "configs[4]":
        rng = np.random.default_rng(2)
        sched = [[int(rng.integers(0, 256)) if (T + s) % 7 in (0, 1, 2) else None for s in range(steps)]
                 for _ in range(n)]
    engine = Engine(model)
    greedy = TemperatureSampler(0.0)
    kw = dict(num_samples=1, max_tokens=steps, sampler=greedy, force_schedule=sched)
    engine.generate_multi_batch(prompts, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    results, _ = engine.generate_multi_batch(prompts, **kw)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    assert len(results) == n and len(results[0]) == T + steps
    out = {"workload": f"{name} end to end through Engine.generate_multi_batch: GPT(n_embd={C}, n_head={H}, "
                       f"n_layer={L}) bf16, {n} prompts x {T} tokens, {steps} decode steps"
                       + (", force_schedule per prompt (channels 0-2 of 7)" if sched else ", greedy"),
           "seconds": el, "generated_tokens_per_s": n * steps / el}
    del model, engine
    torch.cuda.empty_cache()
    return out


def engine_leg(dtype_name: str, per_series: bool = True):
    """configs[1] end to end through the drop-in API: the README GPT (random
    init, seed 0), 64 series of 96 uniform ids, each one
    Engine.generate_batch(prompt, num_samples=100, max_tokens=48) with a
    temperature-1 sampler -- the reference's call pattern (diff_gpt.py:229-235).
    Includes the non-attention model work (projections, FFN, Block-AttnRes,
    lm_head), sampling and the host-side result lists.  Also one batched call
    with all 6400 rows on one prompt.  per_series=False skips the 64 calls
    (the batched call alone, e.g. under a kernel trace)."""
    import torch

    from diff_gpt.model.engine import Engine
    from diff_gpt.model.gpt import GPT
    from diff_gpt.sampler.temperature import TemperatureSampler

    dev = torch.device("cuda:0")
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=138, n_head=HEADS, n_layer=LAYERS,
                use_checkpoint=False).eval().to(dev).to(dt)
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, 256, (PREFIX,), generator=g).tolist() for _ in range(SERIES)]
    engine = Engine(model)
    sampler = TemperatureSampler(1.0)
    series_s = None
    if per_series:
        engine.generate_batch(prompts[0], num_samples=TRAJ, max_tokens=NEW, sampler=sampler)  # warm-up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s, prompt in enumerate(prompts):
            engine.generate_batch(prompt, num_samples=TRAJ, max_tokens=NEW, sampler=sampler, seed=s)
        torch.cuda.synchronize()
        series_s = time.perf_counter() - t0
    # the whole job as one call: 64 prompts x 100 trajectories, one decode
    # loop; the median of 5 calls after the capturing one, from a collected
    # heap (each call builds 12800 Python lists, and a full garbage
    # collection that one call happens to trigger costs as much as the call)
    engine.generate_multi_batch(prompts, num_samples=TRAJ, max_tokens=NEW, sampler=sampler)  # capture
    torch.cuda.synchronize()
    gc.collect()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        engine.generate_multi_batch(prompts, num_samples=TRAJ, max_tokens=NEW, sampler=sampler)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    multi = statistics.median(times)
    tokens = SERIES * TRAJ * NEW
    return {
        "workload": "configs[1] through the Engine: 64 series x 100 trajectories, 96-token prompts, "
                    "48 temperature-1 steps, README GPT (2 layers, d64, h4); tokens_per_s: one "
                    "generate_multi_batch call (one prefill of the 64 prompts, one decode loop over the "
                    "6400 rows, each series' prompt cache stored once), median of 5 calls",
        "dtype": dtype_name,
        "tokens_per_s": tokens / multi,
        "seconds": multi,
        "seconds_min_max": [min(times), max(times)],
        "per_series_calls_tokens_per_s": None if series_s is None else tokens / series_s,
        "per_series_calls_seconds": series_s,
    }


def engine_cpu_baseline(dtype_name: str, runs: int = 5):
    """The reference's engine pattern on the host cores (oracle.torch_ref) for
    one configs[1] series: a batch-1 prefill, the cache broadcast to 100 rows,
    48 steps of softmax + multinomial and a 100-row forward.  One warm-up
    series, then `runs` series; tokens/s from the median series time (the 64
    series of the job cost the same)."""
    import torch

    from diff_gpt.model.gpt import GPT
    from oracle import torch_ref as tr

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    torch.manual_seed(0)
    model = GPT(vocab_size=256, n_embd=64, block_size=138, n_head=HEADS, n_layer=LAYERS, use_checkpoint=False)
    p = {k: v.detach().to(dt) for k, v in model.state_dict().items()}
    cfg = tr.ModelConfig(vocab_size=256, n_embd=64, block_size=138, n_head=HEADS, n_layer=LAYERS)
    table = tr.freqs_table(HEAD_DIM, 2 * 138, 10000)
    g = torch.Generator().manual_seed(1)

    def series(seed):
        prompt = torch.randint(0, 256, (1, PREFIX), generator=g)
        pc = tr.RefCache(1, HEADS, PREFIX, HEAD_DIM, LAYERS)
        logits = tr.forward(p, cfg, prompt, pc, table)[:, -1].expand(TRAJ, -1)
        cache = tr.RefCache(TRAJ, HEADS, PREFIX + NEW, HEAD_DIM, LAYERS)
        cache.broadcast_from(pc)
        rng = torch.Generator().manual_seed(seed)
        for _ in range(NEW):
            nxt = torch.multinomial(torch.softmax(logits.float(), -1), 1, generator=rng)
            logits = tr.forward(p, cfg, nxt, cache, table)[:, -1]

    ts = []
    with torch.no_grad():
        series(0)
        for s in range(runs):
            t0 = time.perf_counter()
            series(s + 1)
            ts.append(time.perf_counter() - t0)
    med = sorted(ts)[len(ts) // 2]
    return {
        "value": TRAJ * NEW / med,
        "unit": "tokens/s",
        "cores": threads,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"{runs} configs[1] series after a warm-up (100 trajectories x 48 steps each), {dtype_name}, "
                  f"oracle.torch_ref model on the host cores; median {med:.2f} s per series",
    }


def cpu_baseline(dtype_name: str, runs: int = 5):
    """The oracle's torch-CPU restatement of the reference decode path
    (rope.py, rms_norm.py, kv_cache.py insert, mha.py:68 SDPA) on the same
    configs[1] shapes -- 6400 rows, both layers -- at decode steps spread over
    the job (L_kv 97 .. 144): one warm-up step, then each sampled step `runs`
    times; per sampled step the median; tokens/s = 6400 / mean of the
    medians (the job's steps cost about linearly in L_kv, so the sampled mean
    stands for the job's)."""
    import torch

    from oracle import torch_ref as tr

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    B, H, D, L = SERIES * TRAJ, HEADS, HEAD_DIM, LAYERS
    g = torch.Generator().manual_seed(0)
    data = torch.randn((L, 2, B, H, PREFIX + NEW, D), generator=g).to(dt)
    table = tr.freqs_table(D, 2 * 138, 10000).to(dt)
    proj = [(torch.randn((B, 1, H, D), generator=g).to(dt) for _ in range(3)) for _ in range(L)]
    proj = [tuple(p) for p in proj]

    def step(s):
        cache = tr.RefCache(B, H, PREFIX + NEW, D, L)
        cache.data = data
        cache.pos = PREFIX + s
        fc = table[PREFIX + s:PREFIX + s + 1].view(1, 1, 1, -1, 2)
        for layer in range(L):
            q, k, v = proj[layer]
            q, k = tr.rms(tr.rope(q, fc)), tr.rms(tr.rope(k, fc))
            kk, vv = cache.insert(layer, k.transpose(1, 2), v.transpose(1, 2))
            tr.sdpa(q.transpose(1, 2), kk, vv).transpose(1, 2).contiguous()

    sampled = [0, 12, 24, 36, 47]
    meds = []
    with torch.no_grad():
        step(0)
        for s in sampled:
            ts = []
            for _ in range(runs):
                t0 = time.perf_counter()
                step(s)
                ts.append(time.perf_counter() - t0)
            meds.append(sorted(ts)[len(ts) // 2])
    per_step = sum(meds) / len(meds)
    return {
        "value": B / per_step,
        "unit": "tokens/s",
        "cores": threads,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"configs[1] {dtype_name}: decode steps {sampled} of 48 (both layers, 6400 seqs), "
                  f"median of {runs} per step after a warm-up, torch CPU restatement (oracle.torch_ref); "
                  f"{per_step * 1e3:.1f} ms per step",
    }


def calib_copy(nbytes: int = 1 << 30, reps: int = 3):
    """A plain device copy of known size: rocprofv3's FETCH_SIZE / WRITE_SIZE
    for it (ideally nbytes each) give the scale factor of those counters."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calib copy: {reps} x {nbytes} bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--dtype", default="fp32", choices=["fp32", "bf16"])
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-engine", action="store_true", help="skip the end-to-end Engine leg")
    ap.add_argument("--no-shapes", action="store_true",
                    help="skip the attention-alone leg at configs[3] / configs[4] shapes")
    ap.add_argument("--shapes-only", action="store_true",
                    help="run only that leg and print its JSON list")
    ap.add_argument("--traffic-json", default=str(REPO / "profiles" / "decode_attn_cfg1_traffic.json"))
    ap.add_argument("--single-dtype", action="store_true", help="skip the other-dtype decode leg")
    ap.add_argument("--decode-mode", default="shared", choices=["shared", "plain"],
                    help="shared: each series' prefix is read from its first row (what KVCache.prefill "
                         "+ MultiHeadAttention do); plain: every row reads its own copy")
    ap.add_argument("--single-mode", action="store_true", help="skip the other decode-mode leg")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run a 1 GiB device copy (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--engine-only", action="store_true",
                    help="run only the engine leg's one-call configs[1] job (twice: capture, then timed) "
                         "and print its JSON")
    ap.add_argument("--jobs-only", action="store_true",
                    help="run only the configs[3] / configs[4] decode-job legs (captured dg_decode_step launches) "
                         "and print their JSON list")
    ap.add_argument("--e2e-only", choices=["configs[3]", "configs[4]"],
                    help="run only that configuration end to end through Engine.generate_multi_batch "
                         "(warm-up call, then the timed call) and print its JSON")
    ap.add_argument("--no-jobs", action="store_true",
                    help="skip the configs[3] / configs[4] whole-job legs (decode jobs and end-to-end Engine)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (no multi-GPU path); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    if args.calib_copy:
        calib_copy()
    if args.shapes_only:
        print(json.dumps(shapes_leg()), flush=True)
        return
    if args.engine_only:
        print(json.dumps(engine_leg(args.dtype, per_series=False)), flush=True)
        return
    if args.jobs_only:
        print(json.dumps([decode_job_leg(name) for name in DECODE_JOBS]), flush=True)
        return
    if args.e2e_only:
        print(json.dumps(engine_multi_leg(args.e2e_only)), flush=True)
        return
    shared = args.decode_mode == "shared"
    res = decode_job(args.dtype, args.steps, args.warmup, shared)
    log(f"decode {args.dtype} {args.decode_mode}: {res}")
    res_mode = None
    if not args.single_mode:
        res_mode = decode_job(args.dtype, max(1, args.steps // 2), 1, not shared)
        log(f"decode {args.dtype} {'plain' if shared else 'shared'}: {res_mode}")
    other = "bf16" if args.dtype == "fp32" else "fp32"
    res_other = None
    if not args.single_dtype:
        res_other = decode_job(other, max(1, args.steps // 2), 1, shared)
        log(f"decode {other} {args.decode_mode}: {res_other}")
    res_unfused = None
    if not args.single_mode:
        # the same job as two launches per layer-step (RoPE/append, then attention)
        res_unfused = decode_job(args.dtype, max(1, args.steps // 2), 1, shared, fused=False)
        log(f"decode {args.dtype} {args.decode_mode} unfused: {res_unfused}")
    traffic = None
    tp = Path(args.traffic_json)
    if tp.exists():
        tj = json.loads(tp.read_text())
        traffic = tj.get(args.dtype + ("_shared" if shared else ""))
    roof = {
        "bound": "hbm",
        "achieved": res["achieved_gbs"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": res["achieved_gbs"] / HBM_PEAK_GBS,
        "traffic": traffic,
    }
    prefill = None if args.no_prefill else prefill_leg(traffic_json=args.traffic_json)
    if prefill:
        log(f"prefill: {prefill}")
        if not args.no_cpu_baseline:
            prefill["cpu_baseline"] = prefill_cpu_baseline()
            log(f"prefill cpu: {prefill['cpu_baseline']}")
    shapes = None if args.no_shapes else shapes_leg()
    jobs = None
    if not args.no_jobs:
        jobs = []
        for name in DECODE_JOBS:
            jobs.append(decode_job_leg(name))
            log(f"job: {jobs[-1]}")
        for name in DECODE_JOBS:
            jobs.append(engine_multi_leg(name))
            log(f"job: {jobs[-1]}")
    engine = None if args.no_engine else engine_leg(args.dtype)
    if engine:
        log(f"engine: {engine}")
        if not args.no_cpu_baseline:
            engine["cpu_baseline"] = engine_cpu_baseline(args.dtype)
            log(f"engine cpu: {engine['cpu_baseline']}")
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.dtype)
    out = {
        "metric": METRIC,
        "value": res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.dtype == "fp32" else "bf16",
        "data": "synthetic (seeded randn q/k/v and KV prefix, resident in HBM)",
        "config": {
            "workload": "configs[1]: 6400 seqs (64 series x 100 trajectories), 96-token prefix, "
                        "48 decode steps, 2 layers, H=4, D=16; step = whole 48-token decode job "
                        "(fused RoPE+QK-norm+append + decode attention per layer-step)",
            "sequences": SERIES * TRAJ,
            "decode_steps": NEW,
            "kv_len": [PREFIX + 1, PREFIX + NEW],
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "decode_kernel": {"mean_us": res["kernel_mean_us"], "bytes_per_launch": res["bytes_per_launch"],
                          "attn_only_tokens_per_s": res["attn_only_tokens_per_s"]},
        "decode_mode": args.decode_mode,
        "decode_other_mode": None if res_mode is None else {
            "mode": "plain" if shared else "shared", "tokens_per_s": res_mode["tokens_per_s"],
            "kernel_mean_us": res_mode["kernel_mean_us"],
            "achieved_gbs": res_mode["achieved_gbs"], "frac": res_mode["achieved_gbs"] / HBM_PEAK_GBS},
        "decode_unfused": None if res_unfused is None else {
            "tokens_per_s": res_unfused["tokens_per_s"], "ms_per_step": res_unfused["ms_per_step"],
            "attention_kernel_mean_us": res_unfused["kernel_mean_us"],
            "attention_achieved_gbs": res_unfused["achieved_gbs"],
            "attention_frac": res_unfused["achieved_gbs"] / HBM_PEAK_GBS},
        "decode_other_dtype": None if res_other is None else {
            "dtype": other, "tokens_per_s": res_other["tokens_per_s"],
            "kernel_mean_us": res_other["kernel_mean_us"],
            "achieved_gbs": res_other["achieved_gbs"],
            "frac": res_other["achieved_gbs"] / HBM_PEAK_GBS},
        "prefill": prefill,
        "shapes": shapes,
        "jobs": jobs,
        "engine": engine,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
