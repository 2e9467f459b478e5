"""dg_decode_step_noalloc (the decode step whose key-split partials live in
the library's static device scratch) against dg_decode_step with a
caller-allocated workspace, through the C-ABI.

Both run the same kernels with the same number of key splits, so the cache
writes and the attention output are compared bit for bit.  Two calls in a
row, the second smaller than the first (the scratch keeps the first call's
partials, which the second must not see), then the device-position form and
a shared-prefix step, and that no size's split workspace exceeds the
scratch (host-side sizing, no GPU work)."""

import ctypes

import pytest
import torch

from oracle import numerics as on  # noqa: F401  (tests share the oracle import path)

CASES = [  # (B, H, D, dtype, max_pos, pos, group, prefix_len)
    (4, 8, 128, torch.bfloat16, 3200, 3000, 1, 0),  # configs[4]-like rows: 25 key splits
    (2, 4, 64, torch.float32, 2600, 2400, 1, 0),    # smaller second call: 20 splits
    (1, 2, 1000, torch.bfloat16, 5000, 4800, 1, 0),  # head_dim 1000 (pair slices): 39 splits
]


def _inputs(dev, B, H, D, dtype, max_pos, seed):
    from diff_gpt.model.rope import precompute_freqs_cis

    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v = (torch.randn((B, 1, H, D), generator=g, device=dev).to(dtype) for _ in range(3))
    cache = torch.randn((2, B, H, max_pos, D), generator=g, device=dev).to(dtype)
    table = precompute_freqs_cis(D, max_pos, 10000).to(dev).to(dtype)
    return q, k, v, cache, table


def _step(dev, case, seed, noalloc, device_pos=False):
    from diff_gpt import _native

    B, H, D, dtype, max_pos, pos, group, prefix = case
    q, k, v, cache, table = _inputs(dev, B, H, D, dtype, max_pos, seed)
    y = torch.empty_like(q)
    kc, vc = cache[0].transpose(1, 2), cache[1].transpose(1, 2)
    if device_pos:
        p, freqs = torch.tensor([pos], dtype=torch.int32, device=dev), table
    else:
        p, freqs = pos, table[pos]
    _native.decode_step_(q, k, v, freqs, kc, vc, y, D ** -0.5, p, prefix, group, noalloc=noalloc)
    torch.cuda.synchronize()
    return y, cache


@pytest.mark.gpu
def test_noalloc_decode_step_equals_workspace_form(dev):
    from diff_gpt import _native

    lib = _native.lib()
    for case in CASES:
        B, H, D, dtype, max_pos, _, _, _ = case
        code = {torch.float32: 0, torch.bfloat16: 1}[dtype]
        need = lib.dg_decode_step_workspace_size(B, H, max_pos, D, code)
        assert 0 < need <= lib.dg_decode_step_noalloc_scratch_bytes()  # the scratch is used
    for i, case in enumerate(CASES):  # large call, then a smaller one
        print(f"noalloc case {i}: {case}", flush=True)
        y1, c1 = _step(dev, case, 10 + i, noalloc=True)
        y0, c0 = _step(dev, case, 10 + i, noalloc=False)
        assert torch.equal(c1, c0), i
        assert torch.equal(y1, y0), i
    # device-position form (graph-replayable), after the two calls above
    y1, c1 = _step(dev, CASES[0], 20, noalloc=True, device_pos=True)
    y0, c0 = _step(dev, CASES[0], 20, noalloc=False, device_pos=True)
    assert torch.equal(c1, c0) and torch.equal(y1, y0)
    # shared-prefix step (one fused launch, no scratch involved)
    shared = (32, 4, 16, torch.float32, 144, 120, 32, 96)
    y1, c1 = _step(dev, shared, 30, noalloc=True)
    y0, c0 = _step(dev, shared, 30, noalloc=False)
    assert torch.equal(c1, c0) and torch.equal(y1, y0)


def test_noalloc_scratch_covers_every_decode_step():
    """Key splits beyond the 16 that one workgroup merges (8 for head dims
    past 512) occur only while B*H < 256 (512), so at most 4351 partials of
    padded head_dim + 2 <= 514 floats (4607 of <= 1026) need the scratch:
    every decode step fits the 20 MiB array (host-side sizing, so this runs
    without a GPU).  The workspace-size query agrees with that bound over a
    sweep of row counts, lengths and head sizes."""
    from diff_gpt import _native

    lib = _native.lib()
    cap = lib.dg_decode_step_noalloc_scratch_bytes()
    assert cap == 20 << 20
    worst = 0
    for bh in list(range(1, 300)) + [383, 511, 512, 1024, 2047, 4095, 4096, 8191, 100000]:
        for max_pos in (1, 255, 256, 2175, 2176, 4096, 8192, 65536, 1 << 20):
            for D in (16, 64, 128, 256, 300, 512, 1000, 1024):
                need = lib.dg_decode_step_workspace_size(bh, 1, max_pos, D, 1)
                assert need <= cap, (bh, max_pos, D, need)
                if need:
                    assert bh < (256 if D <= 512 else 512), (bh, max_pos, D)
                    assert need <= (4351 * 514 if D <= 512 else 4607 * 1026) * 4, (bh, max_pos, D, need)
                worst = max(worst, need)
    assert 0 < worst <= 4607 * 1026 * 4
