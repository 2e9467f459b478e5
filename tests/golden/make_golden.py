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
    ``force_schedule``: token ids and masks.

Outputs: gpt_weights.json, gpt_forward.npz, engine_greedy.json (all small).
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

    (OUT / "gpt_weights.json").write_text(json.dumps(weights, indent=1) + "\n")
    np.savez_compressed(OUT / "gpt_forward.npz", **arrays)
    (OUT / "engine_greedy.json").write_text(json.dumps(engine_doc, indent=1) + "\n")
    print("wrote", sorted(p.name for p in OUT.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
