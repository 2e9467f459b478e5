"""KV-cache generation engine (src/diff_gpt/model/engine.py:11-169).

One batch-1 prefill of the prompt, a broadcast of its KV cache to
``num_samples`` rows (KVCache.prefill), then one single-token decode forward
per step for all rows together.  Per step a token column is either sampled
(``sampler`` or softmax + multinomial with the seeded device generator) or,
when ``force_schedule[step]`` is an int, forced for every row.  Each yielded
column comes with a mask column: 1 = sampled, 0 = forced.
"""

from collections import deque
from typing import Generator

import torch

from diff_gpt.model.gpt import BaseGPT
from diff_gpt.model.kv_cache import KVCache
from diff_gpt.sampler.sampler import Sampler


class RowState:
    """Per-row generation state: the tokens so far and a queue of tokens that
    must be emitted next regardless of sampling (engine.py:11-20)."""

    __slots__ = (
        "current_tokens",
        "forced_tokens",
    )

    def __init__(self, current_tokens: list[int] | None = None) -> None:
        self.current_tokens = current_tokens or list()
        self.forced_tokens = deque()


class Engine:
    __slots__ = "model"

    def __init__(self, model: BaseGPT) -> None:
        self.model = model

    def _budget(self, prompt_len: int, max_tokens: int | None) -> int:
        # RoPE table covers 2*block_size positions (engine.py:55-64)
        ceiling = max(0, self.model.block_size * 2 - prompt_len)
        return ceiling if max_tokens is None else min(max_tokens, ceiling)

    @torch.inference_mode()
    def generate(
        self,
        tokens: list[int],
        num_samples: int = 1,
        max_tokens: int | None = None,
        sampler: Sampler | None = None,
        seed: int = 42,
        force_schedule: list[int | None] | None = None,
    ) -> Generator[tuple[list[int], list[int]], None, None]:
        """
        Streaming generation: single prefill, then clone the KV cache for each sample.

        `force_schedule`, when provided, is a per-step list aligned with the
        generation loop: `None` samples at that step, an `int` teacher-forces
        that token for every row.  Its length must be at least the number of
        generated steps.
        """
        assert isinstance(tokens, list), "tokens must be a list of ints"
        assert len(tokens) > 0, "tokens must be non-empty"
        assert all(isinstance(t, int) for t in tokens), "tokens must be a list of ints"

        steps = self._budget(len(tokens), max_tokens)
        if steps == 0:
            return
        if force_schedule is not None:
            assert len(force_schedule) >= steps, (
                f"force_schedule must cover all generation steps "
                f"(len={len(force_schedule)} < {steps})"
            )

        model = self.model
        device = model.device_type
        rng = torch.Generator(device=device)
        rng.manual_seed(seed)
        geometry = {
            "num_heads": model.n_head,
            "head_dim": model.n_embd // model.n_head,
            "num_layers": model.n_layer,
        }

        # 1) batch-1 prefill of the prompt
        prompt_cache = KVCache(batch_size=1, seq_len=len(tokens), **geometry)
        ids = torch.tensor([tokens], dtype=torch.long, device=device)
        logits, _ = model.forward(ids, kv_cache=prompt_cache)
        logits = logits[:, -1, :].expand(num_samples, -1)

        # 2) every row starts from the same prompt cache
        cache = KVCache(batch_size=num_samples, seq_len=len(tokens) + steps, **geometry)
        cache.prefill(prompt_cache)
        del prompt_cache

        rows = [RowState(list(tokens)) for _ in range(num_samples)]

        for step in range(steps):
            forced = None if force_schedule is None else force_schedule[step]
            if forced is None:
                if sampler is not None:
                    picked = sampler(logits, rng=rng)
                else:
                    picked = torch.multinomial(
                        torch.softmax(logits, dim=-1), num_samples=1, generator=rng
                    )
                proposals = picked[:, 0].tolist()
            else:
                proposals = [forced] * num_samples

            column: list[int] = []
            masks: list[int] = []
            for row, proposal in zip(rows, proposals):
                queued = len(row.forced_tokens) > 0
                tok = row.forced_tokens.popleft() if queued else proposal
                masks.append(0 if (queued or forced is not None) else 1)
                column.append(tok)
                row.current_tokens.append(tok)
            yield column, masks

            # 3) one decode forward for the column just emitted
            ids = torch.tensor(column, dtype=torch.long, device=device).unsqueeze(1)
            logits, _ = model.forward(ids, kv_cache=cache)
            logits = logits[:, -1, :]

    def generate_batch(
        self, tokens: list[int], num_samples: int = 1, **kwargs
    ) -> tuple[list[list[int]], list[list[int]]]:
        """
        Non-streaming batch generation that just returns the final token sequences.
        Returns (results, masks): each a list of `num_samples` lists of ints.
        """
        results = [list(tokens) for _ in range(num_samples)]
        masks = [[0] * len(tokens) for _ in range(num_samples)]
        for column, mask_column in self.generate(tokens, num_samples, **kwargs):
            for res, m, tok, mk in zip(results, masks, column, mask_column):
                res.append(tok)
                m.append(mk)
        return results, masks
