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


class _DecodeGraph:
    """GPT.forward over one new token per row, captured once as a HIP graph and
    replayed for every decode step.

    The cache carries a device copy of its position (KVCache.pos_dev); the
    attention layers then launch the position-reading kernels
    (dg_rope_qknorm_append_at, dg_decode_attention_at) and the model hands
    them the whole RoPE table, so nothing in the captured launches depends on
    the step.  The graph ends by advancing pos_dev; step() advances the host
    copy.  Inputs go through a static id buffer, the logits come back in a
    static buffer that the next replay overwrites."""

    __slots__ = ("cache", "ids", "graph", "logits")

    def __init__(self, model: BaseGPT, cache: KVCache, n_rows: int, device: torch.device) -> None:
        self.cache = cache
        self.ids = torch.zeros((n_rows, 1), dtype=torch.long, device=device)
        pos0 = cache.pos
        cache.pos_dev = torch.full((1,), pos0, dtype=torch.int32, device=device)
        try:
            # warm-up outside the capture (library handles, allocator); it
            # appends the K/V of a zero token at pos0, which the first replay
            # overwrites
            side = torch.cuda.Stream(device=device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                model.forward(self.ids, kv_cache=cache)
            torch.cuda.current_stream(device).wait_stream(side)
            cache.pos = pos0
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                logits, _ = model.forward(self.ids, kv_cache=cache)
                self.logits = logits[:, -1, :]
                cache.pos_dev.add_(1)
            cache.pos = pos0
        except BaseException:
            cache.pos = pos0
            cache.pos_dev = None
            raise

    def step(self, ids: torch.Tensor) -> torch.Tensor:
        self.ids.copy_(ids)
        self.graph.replay()
        self.cache.pos += 1
        return self.logits

    def rewind(self) -> None:
        """Start over at the cache's (refilled) host position."""
        self.cache.pos_dev.fill_(self.cache.pos)

    def close(self) -> None:
        self.cache.pos_dev = None


# A captured decode step (and the cache it writes) is kept for the next call
# when the cache is at most this large.
_KEEP_GRAPH_BYTES = 1 << 30


class Engine:
    __slots__ = ("model", "use_graph", "_kept")

    def __init__(self, model: BaseGPT, use_graph: bool = True) -> None:
        """use_graph: replay the decode step as a captured HIP graph (same
        kernels and arithmetic as the eager forward, no per-step launch
        overhead); False runs every step eagerly.  The captured step and its
        cache (up to 1 GiB) are kept after a call and reused by the next call
        with the same rows, prompt length and budget while the model's
        parameters are unchanged (same storage, no in-place update)."""
        self.model = model
        self.use_graph = use_graph
        self._kept = None  # (key, cache, _DecodeGraph), free for the next call

    def _graph_key(self, num_samples: int, prompt_len: int, steps: int) -> tuple:
        model = self.model
        params = tuple((p.data_ptr(), p._version) for p in model.parameters())
        buffers = tuple(b.data_ptr() for b in model.buffers())
        return (id(model), num_samples, prompt_len, steps, params, buffers)

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
        # The per-row forcing queues of RowState are never filled inside a
        # generation call (engine.py:129-144 passes the sampled or scheduled
        # column through), so a column is the sampled/forced tokens and its
        # mask is 1 for a sampled step, 0 for a forced one.
        for column, forced in self._device_steps(
            tokens, num_samples, max_tokens, sampler, seed, force_schedule
        ):
            yield column.tolist(), [0 if forced else 1] * num_samples

    def _device_steps(
        self,
        tokens: list[int],
        num_samples: int,
        max_tokens: int | None,
        sampler: Sampler | None,
        seed: int,
        force_schedule: list[int | None] | None,
    ) -> Generator[tuple[torch.Tensor, bool], None, None]:
        """The generation loop with the token columns kept on the device:
        yields ((num_samples,) int64 column, forced) per step, and feeds each
        column to the next decode forward without a host round trip."""
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

        # 2) every row starts from the same prompt cache (read once per
        #    decode step thanks to the recorded shared prefix); a step captured
        #    by an earlier call with the same key replays into its own cache
        use_graph = self.use_graph and steps > 1 and torch.device(device).type == "cuda"
        key = self._graph_key(num_samples, len(tokens), steps) if use_graph else None
        kept, self._kept = self._kept, None  # taken: a concurrent call builds its own
        decode = None
        if kept is not None and kept[0] == key:
            _, cache, decode = kept
            cache._refill(prompt_cache)
            decode.rewind()
        else:
            if kept is not None:
                kept[2].close()
            cache = KVCache(batch_size=num_samples, seq_len=len(tokens) + steps, **geometry)
            cache.prefill(prompt_cache)
            if use_graph:
                decode = _DecodeGraph(model, cache, num_samples, torch.device(device))
        del prompt_cache

        try:
            for step in range(steps):
                forced = None if force_schedule is None else force_schedule[step]
                if forced is None:
                    if sampler is not None:
                        picked = sampler(logits, rng=rng)
                    else:
                        picked = torch.multinomial(
                            torch.softmax(logits, dim=-1), num_samples=1, generator=rng
                        )
                    column = picked[:, 0]
                else:
                    column = torch.full((num_samples,), forced, dtype=torch.long, device=logits.device)
                yield column, forced is not None

                # 3) one decode forward for the column just emitted
                ids = column.unsqueeze(1)
                if decode is not None:
                    logits = decode.step(ids)
                else:
                    logits, _ = model.forward(ids, kv_cache=cache)
                    logits = logits[:, -1, :]
        finally:
            if decode is not None:
                if cache.nbytes() <= _KEEP_GRAPH_BYTES:
                    self._kept = (key, cache, decode)
                else:
                    decode.close()

    @torch.inference_mode()
    def generate_batch(
        self, tokens: list[int], num_samples: int = 1, **kwargs
    ) -> tuple[list[list[int]], list[list[int]]]:
        """
        Non-streaming batch generation that just returns the final token sequences.
        Returns (results, masks): each a list of `num_samples` lists of ints.
        """
        unknown = set(kwargs) - {"max_tokens", "sampler", "seed", "force_schedule"}
        if unknown:
            raise TypeError(f"generate() got unexpected keyword arguments {sorted(unknown)}")
        columns, mask_steps = [], []
        for column, forced in self._device_steps(
            tokens,
            num_samples,
            kwargs.get("max_tokens"),
            kwargs.get("sampler"),
            kwargs.get("seed", 42),
            kwargs.get("force_schedule"),
        ):
            columns.append(column)
            mask_steps.append(0 if forced else 1)
        generated = torch.stack(columns, dim=1).tolist() if columns else [[] for _ in range(num_samples)]
        results = [list(tokens) + row for row in generated]
        masks = [[0] * len(tokens) + mask_steps for _ in range(num_samples)]
        return results, masks
