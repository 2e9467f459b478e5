"""Write the golden vectors of tests/golden/ from the reference implementation.

Run in the build container only (the reference is not present on GPU hosts):

    python tests/golden/make_golden.py /root/reference/src

It imports fxeqxmulfx/diff-gpt's own ``diff_gpt`` package from the given
source directory (never this repository's package of the same name) and
records, on the CPU, what no closed form or known-answer test pins:

  * seed -> weights: the state_dict of ``GPT(...)`` built under
    ``torch.manual_seed(0)`` (gpt.py:117-130, mha.py:25-29,
    feed_forward.py:10-14, block.py:71-72), as a SHA-256 over the fp32 bytes
    in key order plus a few leading values per tensor;
  * the end-to-end composition of ``GPT.forward`` (gpt.py:140-200 with
    Block-AttnRes block.py:10-107): full-forward logits, and the KV-cache
    prefill + greedy decode loop driven as tests/diff_gpt/model/test_gpt.py:34-76
    does (tokens, per-step logits, final cache contents);
  * ``Engine.generate_batch`` (engine.py:29-169) with a greedy sampler and a
    ``force_schedule``: token ids and masks;
  * the sigma-delta tokenizer (encoder_decoder.py:278-427) on small seeded
    series: encode's (start, scale, tokens), decode(encode(x)) and
    get_domain_of_definition, for shared and per-column orders, the carry,
    MASH and plain-rounding quantisers, float64 and Decimal;
  * the forecasting API (diff_gpt.py:127-505) with a greedy sampler on the
    seeded cfg0 model: predict (autoregressive and teacher-forced),
    predict_samples, predict_quantiles, anomaly_scores.

Outputs: gpt_weights.json, gpt_forward.npz, engine_greedy.json, codec.json,
diffgpt.json (all small).
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent

# (name, GPT kwargs, prompt shape, decode steps)
MODELS = [
    ("cfg0", dict(vocab_size=256, n_embd=64, block_size=138, n_head=4, n_layer=2), (2, 8), 4),
    ("lpb2", dict(vocab_size=64, n_embd=32, block_size=20, n_head=4, n_layer=3,
                  attn_res_layers_per_block=2), (2, 7), 3),
]


def _import_reference(src: str):
    sys.path.insert(0, src)
    import diff_gpt  # noqa: F401

    where = Path(diff_gpt.__file__).resolve()
    if not str(where).startswith(str(Path(src).resolve())):
        raise SystemExit(f"imported diff_gpt from {where}, not from {src}")
    from diff_gpt.model.engine import Engine
    from diff_gpt.model.gpt import GPT
    from diff_gpt.model.kv_cache import KVCache
    from diff_gpt.sampler.temperature import TemperatureSampler

    return GPT, KVCache, Engine, TemperatureSampler


# (name, seed, rows, cols, vocab, order, use_decimal); a list order is per column
CODEC_CASES = [
    ("k0_f64", 1, 12, 2, 256, 0, False),
    ("k1_f64", 2, 20, 3, 256, 1, False),
    ("k2_mash_f64", 3, 25, 2, 256, 2, False),
    ("k3_mash_f64", 4, 25, 2, 64, 3, False),
    ("k3_small_vocab_carry_f64", 5, 16, 2, 8, 3, False),
    ("k4_mash_dec", 6, 18, 2, 256, 4, True),
    ("k1_dec", 7, 10, 2, 64, 1, True),
    ("percol_f64", 8, 22, 3, 256, [0, 2, 1], False),
    ("percol_dec", 9, 14, 3, 128, [3, 0, 1], True),
]


def _series(seed: int, rows: int, cols: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    t = np.arange(rows, dtype=np.float64)[:, None]
    base = np.sin(t * (0.3 + 0.1 * np.arange(cols))) * (1 + np.arange(cols)) + 0.05 * t
    return base + 0.1 * rng.standard_normal((rows, cols))


def _enc(x):
    """JSON form of a codec array: floats as repr, Decimals as str, ints as int."""
    a = np.asarray(x)
    if a.dtype == object:
        return {"decimal": [[str(v) for v in row] for row in a.reshape(a.shape[0], -1)] if a.ndim > 1
                else [str(v) for v in a], "shape": list(a.shape)}
    if np.issubdtype(a.dtype, np.integer):
        return {"int": a.tolist(), "shape": list(a.shape)}
    return {"float": [repr(float(v)) for v in a.reshape(-1)], "shape": list(a.shape)}


def codec_vectors(src: str) -> dict:
    from diff_gpt import encoder_decoder as ed

    out = {}
    for name, seed, rows, cols, vocab, order, dec in CODEC_CASES:
        x = _series(seed, rows, cols)
        order_arg = np.asarray(order, dtype=np.int64) if isinstance(order, list) else order
        xin = ed.np_to_decimal(x) if dec else x
        domain = ed.get_domain_of_definition(xin, order_arg, dec)
        start, scale, tokens = ed.encode(xin, vocab, domain, order_arg, dec)
        back = ed.decode(start, scale, tokens, vocab, order_arg, dec)
        out[name] = {
            "seed": seed, "rows": rows, "cols": cols, "vocab": vocab, "order": order,
            "use_decimal": dec, "input": _enc(x), "domain": _enc(domain), "start": _enc(start),
            "scale": _enc(scale), "tokens": _enc(tokens), "decoded": _enc(back),
        }
    return out


def diffgpt_vectors(GPT, TemperatureSampler) -> dict:
    import pandas as pd

    from diff_gpt import encoder_decoder as ed
    from diff_gpt.diff_gpt import DiffGPT

    torch = __import__("torch")
    torch.manual_seed(0)
    model = GPT(use_checkpoint=False, **MODELS[0][1]).eval()
    x = _series(11, 30, 3)
    df = pd.DataFrame(x, columns=["a", "b", "c"])
    greedy = TemperatureSampler(0.0)
    out = {"frame_seed": 11, "rows": 30, "cols": 3}

    dg = DiffGPT(model, 1, ed.get_domain_of_definition(x, 1, False), False)
    out["order"] = 1
    out["predict"] = dg.predict(df, max_new_points=5, sampler=greedy).to_numpy().tolist()
    ctx, fut = df.iloc[:25].reset_index(drop=True), df.iloc[25:].reset_index(drop=True)
    out["predict_forced"] = dg.predict(ctx, future_covariates_df=fut, target_columns=["a"],
                                       sampler=greedy).to_numpy().tolist()
    out["samples"] = dg.predict_samples(df, max_new_points=4, num_samples=3, sampler=greedy).tolist()
    qs = dg.predict_quantiles(df, max_new_points=4, quantiles=(0.1, 0.5, 0.9), num_samples=3,
                              sampler=greedy)
    out["quantiles"] = {str(q): v.to_numpy().tolist() for q, v in qs.items()}
    out["anomaly"] = [[None if np.isnan(v) else v for v in row]
                      for row in dg.anomaly_scores(df).to_numpy().tolist()]

    orders = np.asarray([1, 2, 0], dtype=np.int64)
    xd = ed.np_to_decimal(x)
    dg2 = DiffGPT(model, orders, ed.get_domain_of_definition(xd, orders, True), True)
    out["percol_decimal_orders"] = orders.tolist()
    out["predict_percol_decimal"] = [[float(v) for v in row] for row in
                                     dg2.predict(df, max_new_points=4, sampler=greedy).to_numpy()]
    return out


def weights_digest(state_dict) -> dict:
    h = hashlib.sha256()
    keys, heads = [], {}
    for k, v in state_dict.items():
        a = v.detach().float().contiguous().numpy()
        h.update(k.encode())
        h.update(a.tobytes())
        keys.append([k, list(a.shape)])
        heads[k] = [float(x) for x in a.reshape(-1)[:4]]
    return {"sha256": h.hexdigest(), "keys": keys, "head_values": heads}


def main(src: str) -> None:
    import torch

    GPT, KVCache, Engine, TemperatureSampler = _import_reference(src)
    torch.set_num_threads(1)
    weights, arrays = {}, {}
    for name, kw, (B, T), steps in MODELS:
        torch.manual_seed(0)
        model = GPT(use_checkpoint=False, **kw).eval()
        weights[name] = {"kwargs": kw, **weights_digest(model.state_dict())}
        ids = torch.randint(0, kw["vocab_size"], (B, T), generator=torch.Generator().manual_seed(1))
        H, D, L = kw["n_head"], kw["n_embd"] // kw["n_head"], kw["n_layer"]
        with torch.no_grad():
            full, _ = model(ids)
            cache = KVCache(batch_size=B, num_heads=H, seq_len=T + steps, head_dim=D, num_layers=L)
            logits, _ = model(ids, kv_cache=cache)
            last = logits[:, -1]
            toks, step_logits = [], []
            for _ in range(steps):
                step_logits.append(last)
                nxt = last.argmax(dim=-1)
                toks.append(nxt)
                logits, _ = model(nxt[:, None], kv_cache=cache)
                last = logits[:, -1]
            step_logits.append(last)
        arrays[f"{name}_ids"] = ids.numpy()
        arrays[f"{name}_full_logits"] = full.numpy()
        arrays[f"{name}_prefill_logits"] = model(ids, kv_cache=KVCache(B, H, T, D, L))[0].detach().numpy()
        arrays[f"{name}_greedy_tokens"] = torch.stack(toks, 1).numpy()
        arrays[f"{name}_step_logits"] = torch.stack(step_logits, 1).numpy()
        arrays[f"{name}_cache"] = cache.kv_cache.numpy()
        arrays[f"{name}_cache_pos"] = np.array(cache.get_pos())

    # Engine: greedy sampler (no RNG draws) with teacher forcing on steps 1, 4
    torch.manual_seed(0)
    model = GPT(use_checkpoint=False, **MODELS[0][1]).eval()
    prompt = torch.randint(0, 256, (12,), generator=torch.Generator().manual_seed(2)).tolist()
    schedule = [None, 7, None, None, 3, None]
    engine = Engine(model)
    res, masks = engine.generate_batch(prompt, num_samples=2, max_tokens=6,
                                       sampler=TemperatureSampler(0.0), force_schedule=schedule)
    res_free, masks_free = engine.generate_batch(prompt, num_samples=3, max_tokens=5,
                                                 sampler=TemperatureSampler(0.0))
    engine_doc = {
        "model": "cfg0", "prompt": prompt,
        "forced": {"num_samples": 2, "max_tokens": 6, "force_schedule": schedule,
                   "results": res, "masks": masks},
        "free": {"num_samples": 3, "max_tokens": 5, "results": res_free, "masks": masks_free},
    }

    codec = codec_vectors(src)
    diffgpt = diffgpt_vectors(GPT, TemperatureSampler)

    (OUT / "codec.json").write_text(json.dumps(codec) + "\n")
    (OUT / "diffgpt.json").write_text(json.dumps(diffgpt) + "\n")
    (OUT / "gpt_weights.json").write_text(json.dumps(weights, indent=1) + "\n")
    np.savez_compressed(OUT / "gpt_forward.npz", **arrays)
    (OUT / "engine_greedy.json").write_text(json.dumps(engine_doc, indent=1) + "\n")
    print("wrote", sorted(p.name for p in OUT.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
