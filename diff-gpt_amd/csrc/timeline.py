"""Per-wave phase timeline of the fused decode step at configs[1].

    python diff-gpt_amd/csrc/build.py --timeline      # builds lib/libdgattn_timeline.so
    python diff-gpt_amd/csrc/timeline.py [fp32|bf16 ...]

The workload is one layer-step of bench.py's configs[1] decode job (6400 rows =
64 series x 100 trajectories, H = 4, D = 16, each series' 96-token prefix in
pages of its own, positions 96 + s), run by dg_decode_step as
attn_shared_kernel<T, 16, FUSED>: per (series, 16-row tile, head) one block of
two waves, wave 0 the prefix on MFMA, wave 1 the rows' own keys plus the new
token.  The measurement library's waves stamp the shader clock (s_memtime) at
their phase boundaries:

  wave 1 (own keys): entry | q and the first register sets issued (issue) |
      RoPE, QK-norm, append (rope_append) | rest of the own-key stream
      (stream) | new key and hand-over (handover) | barrier (barrier) | end
  wave 0 (prefix):   entry | q and the first prefix chunks issued (issue) |
      prefix products (prefix) | barrier (barrier) | merge and store (merge)

Stamps are compared only within a block (the two waves share a CU; counters
of different CUs are not aligned).  Printed per step s in {0, 24, 47}: the
product library's time per launch (20 back-to-back launches, HIP events on the
launch stream), the measurement build's, and the median cycles of each phase
over the 1792 blocks; then the graph-launch floor: the time per launch of an
empty kernel of the same grid, 96 launches captured in one HIP graph (the
decode job's launches are graph replays)."""

from __future__ import annotations

import ctypes
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from diff_gpt import _native  # noqa: E402
from diff_gpt.model.rope import precompute_freqs_cis  # noqa: E402

SERIES, TRAJ, H, D, PREFIX, NEW, L = 64, 100, 4, 16, 96, 48, 2
B = SERIES * TRAJ
NBLK = SERIES * ((TRAJ + 15) // 16) * H  # two-wave blocks of the shared kernel
STEPS = (0, 24, 47)


def _load(path: Path) -> ctypes.CDLL:
    h = ctypes.CDLL(str(path))
    for name, (res, args) in _native._SIGNATURES.items():
        if hasattr(h, name):
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
    return h


def measure(dtype_name: str, prod: ctypes.CDLL, tl: ctypes.CDLL) -> dict:
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    prefix = torch.randn((L, 2, SERIES, H, PREFIX, D), generator=g, device=dev).to(dt)
    cache = torch.randn((L, 2, B, H, NEW, D), generator=g, device=dev).to(dt)
    table = precompute_freqs_cis(D, 2 * 138, 10000).to(dev).to(dt)
    qkv = torch.randn((NEW, 3, B, 1, H, D), generator=g, device=dev).to(dt)
    y = torch.empty((B, 1, H, D), dtype=dt, device=dev)
    code = _native._DTYPE_CODE[dt]
    side = torch.cuda.Stream()
    stream = ctypes.c_void_p(side.cuda_stream)
    keep = []

    def args_for(s: int) -> tuple:
        t0 = PREFIX + s
        q, k, v = qkv[s]
        pk, pv = prefix[0, 0].transpose(1, 2), prefix[0, 1].transpose(1, 2)
        pre, _ = _native._prefix_arg(_native.Prefix(PREFIX, TRAJ, pk, pv, PREFIX))
        keep.append(pre)
        kc, vc = cache[0, 0].transpose(1, 2), cache[0, 1].transpose(1, 2)
        st = lambda t: ctypes.pointer(_native._bthd_strides(t))  # noqa: E731
        return (B, H, D, code, _native._ptr(q), st(q), _native._ptr(k), st(k), _native._ptr(v), st(v),
                _native._ptr(kc), st(kc), _native._ptr(vc), st(vc), _native._ptr(table[t0]), 0, code, t0, None,
                PREFIX + NEW, _native._ptr(y), st(y), D ** -0.5, pre, _native.DG_QKNORM, None, 0, stream)

    out = {"dtype": dtype_name, "steps": {}}
    for s in STEPS:
        a = args_for(s)
        us = []
        for lib in (prod, tl):
            with torch.cuda.stream(side):
                for _ in range(3):
                    rc = lib.dg_decode_step(*a)
                    if rc != 0:
                        raise RuntimeError(lib.dg_last_error().decode())
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(side)
                for _ in range(20):
                    lib.dg_decode_step(*a)
                e1.record(side)
            torch.cuda.synchronize()
            us.append(e0.elapsed_time(e1) / 20 * 1e3)
        buf = torch.zeros(NBLK * 2 * 8, dtype=torch.int64, device=dev)
        assert tl.dg_timeline_set(ctypes.c_void_p(buf.data_ptr())) == 0
        with torch.cuda.stream(side):
            tl.dg_decode_step(*a)
        torch.cuda.synchronize()
        assert tl.dg_timeline_set(ctypes.c_void_p(0)) == 0
        t = buf.cpu().numpy().reshape(NBLK, 2, 8).astype(np.int64)
        w0, w1 = t[:, 0], t[:, 1]
        assert (w0[:, 0] > 0).all() and (w1[:, 0] > 0).all(), "a block left no stamps"
        med = lambda x: float(np.median(x))  # noqa: E731
        out["steps"][s] = {
            "product_us": us[0], "timing_build_us": us[1],
            "block_cycles": med(np.maximum(w0[:, 6], w1[:, 6]) - np.minimum(w0[:, 0], w1[:, 0])),
            "w1_issue": med(w1[:, 1] - w1[:, 0]), "w1_rope_append": med(w1[:, 2] - w1[:, 1]),
            "w1_stream": med(w1[:, 3] - w1[:, 2]), "w1_handover": med(w1[:, 4] - w1[:, 3]),
            "w1_barrier": med(w1[:, 5] - w1[:, 4]),
            "w0_issue": med(w0[:, 1] - w0[:, 0]), "w0_prefix": med(w0[:, 2] - w0[:, 1]),
            "w0_barrier": med(w0[:, 5] - w0[:, 2]), "w0_merge": med(w0[:, 6] - w0[:, 5]),
        }
    for blocks, threads in ((NBLK, 128), (1, 64)):
        with torch.cuda.stream(side):
            tl.dg_timeline_empty(blocks, threads, stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for _ in range(96):
                tl.dg_timeline_empty(blocks, threads, cs)
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        out[f"empty_graph_launch_us_{blocks}x{threads}"] = e0.elapsed_time(e1) / 10 / 96 * 1e3
    return out


def report(res: dict) -> str:
    lines = [f"### {res['dtype']}", "",
             f"Empty kernel in a graph: {res[f'empty_graph_launch_us_{NBLK}x128']:.2f} us per launch at "
             f"{NBLK} blocks x 128 threads, {res['empty_graph_launch_us_1x64']:.2f} us at 1 x 64.", "",
             "| s | us/launch (product) | us/launch (timing build) | cycles per block | wave 1: issue | rope+append "
             "| stream | handover | barrier | wave 0: issue | prefix | barrier | merge+store |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for s, r in res["steps"].items():
        lines.append(f"| {s} | {r['product_us']:.2f} | {r['timing_build_us']:.2f} | {r['block_cycles']:.0f} | "
                     f"{r['w1_issue']:.0f} | {r['w1_rope_append']:.0f} | {r['w1_stream']:.0f} | "
                     f"{r['w1_handover']:.0f} | {r['w1_barrier']:.0f} | {r['w0_issue']:.0f} | "
                     f"{r['w0_prefix']:.0f} | {r['w0_barrier']:.0f} | {r['w0_merge']:.0f} |")
    return "\n".join(lines)


def main() -> None:
    prod = _load(_native.LIB_PATH)
    tl_path = _native.LIB_PATH.with_name("libdgattn_timeline.so")
    if not tl_path.exists():
        raise SystemExit(f"{tl_path} not built: python diff-gpt_amd/csrc/build.py --timeline")
    tl = _load(tl_path)
    tl.dg_timeline_set.argtypes = [ctypes.c_void_p]
    tl.dg_timeline_set.restype = ctypes.c_int
    tl.dg_timeline_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    tl.dg_timeline_empty.restype = ctypes.c_int
    results = [measure(d, prod, tl) for d in (sys.argv[1:] or ["bf16", "fp32"])]
    for r in results:
        print(report(r), flush=True)
        print()
    print(json.dumps(results), flush=True)


if __name__ == "__main__":
    main()
