"""KV-cache generation engine (src/diff_gpt/model/engine.py:11-169).

One batch-1 prefill of the prompt, the prompt's KV cache shared by
``num_samples`` rows (KVCache.prefill: stored once, read once per decode
step), then one single-token decode forward per step for all rows together.
Per step a token column is either sampled (``sampler`` or softmax +
multinomial with the seeded device generator) or, when
``force_schedule[step]`` is an int, forced for every row.  Each yielded
column comes with a mask column: 1 = sampled, 0 = forced.

Beyond the reference: ``generate_multi`` / ``generate_multi_batch`` decode
several prompts of one length at once -- one batched prefill, each prompt's
cache shared by its ``num_samples`` rows, one captured decode step for all
rows -- with a schedule that may differ per prompt or per row.
"""

import gc
from collections import deque
from typing import Generator, Sequence

import numpy as np
import torch

from diff_gpt.model.gpt import GPT, BaseGPT
from diff_gpt.model.kv_cache import KVCache
from diff_gpt.sampler.sampler import Sampler
from diff_gpt.sampler.temperature import draw_one


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

# kinds of a decode step's column
_SAMPLE, _FORCE_ALL, _MIXED = 0, 1, 2


class _Schedule:
    """A force schedule resolved for ``rows`` rows over ``steps`` steps: per
    step, whether every row samples, every row is forced, or some are; the
    forced tokens as a (steps, rows) device tensor (negative: sample) when
    they differ between rows, else one token per step."""

    __slots__ = ("kinds", "shared", "per_row")

    def __init__(self, steps: int) -> None:
        self.kinds = [_SAMPLE] * steps
        self.shared: list[int | None] | None = None
        self.per_row: torch.Tensor | None = None

    @staticmethod
    def shared_list(schedule: Sequence[int | None], steps: int) -> "_Schedule":
        s = _Schedule(steps)
        s.shared = list(schedule[:steps])
        s.kinds = [_SAMPLE if t is None else _FORCE_ALL for t in s.shared]
        return s

    @staticmethod
    def table(table: np.ndarray, steps: int, device) -> "_Schedule":
        """table: (rows, >= steps) integers, negative = sample."""
        s = _Schedule(steps)
        t = np.ascontiguousarray(table[:, :steps].T, dtype=np.int64)  # (steps, rows)
        forced = t >= 0
        for i in range(steps):
            if forced[i].all():
                s.kinds[i] = _FORCE_ALL
            elif forced[i].any():
                s.kinds[i] = _MIXED
        s.per_row = torch.from_numpy(t).to(device)
        return s


class Engine:
    __slots__ = ("model", "use_graph", "_kept")

    def __init__(self, model: BaseGPT, use_graph: bool = True) -> None:
        """use_graph: replay the decode step as a captured HIP graph (same
        kernels and arithmetic as the eager forward, no per-step launch
        overhead); False runs every step eagerly.  The captured step and its
        cache (up to 1 GiB) are kept after a call and reused by the next call
        with the same prompts count, rows, prompt length and budget while the
        model's parameters are unchanged (same storage, no in-place update)."""
        self.model = model
        self.use_graph = use_graph
        self._kept = None  # (key, cache, _DecodeGraph), free for the next call

    def _graph_key(self, n_prompts: int, num_samples: int, prompt_len: int, steps: int) -> tuple:
        model = self.model
        params = tuple((p.data_ptr(), p._version) for p in model.parameters())
        buffers = tuple(b.data_ptr() for b in model.buffers())
        return (id(model), n_prompts, num_samples, prompt_len, steps, params, buffers)

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
        self._check_tokens(tokens)
        for column, mask in self._device_steps([tokens], num_samples, max_tokens, sampler, seed,
                                               force_schedule, per_prompt=False):
            yield column.tolist(), _mask_list(mask, num_samples)

    @torch.inference_mode()
    def generate_batch(
        self, tokens: list[int], num_samples: int = 1, **kwargs
    ) -> tuple[list[list[int]], list[list[int]]]:
        """
        Non-streaming batch generation that just returns the final token sequences.
        Returns (results, masks): each a list of `num_samples` lists of ints.
        """
        self._check_tokens(tokens)
        return self._collect([tokens], num_samples, kwargs, per_prompt=False)

    @torch.inference_mode()
    def generate_multi(
        self,
        prompts: list[list[int]],
        num_samples: int = 1,
        max_tokens: int | None = None,
        sampler: Sampler | None = None,
        seed: int = 42,
        force_schedule=None,
    ) -> Generator[tuple[list[int], list[int]], None, None]:
        """Streaming generation for several prompts of one length at once:
        row r = p * num_samples + i is trajectory i of prompt p.  Yields a
        (column, mask) pair of len(prompts) * num_samples ints per step.

        `force_schedule` may be None; one list shared by every row (as in
        generate); a list of per-prompt lists (the rows of a prompt share
        it); or a (rows, steps) integer array with a negative entry where the
        row samples.  A step that forces every row draws nothing from the
        generator; a step where some rows sample draws for all rows and keeps
        the forced tokens where they are scheduled."""
        self._check_prompts(prompts)
        for column, mask in self._device_steps(prompts, num_samples, max_tokens, sampler, seed,
                                               force_schedule, per_prompt=True):
            yield column.tolist(), _mask_list(mask, len(prompts) * num_samples)

    @torch.inference_mode()
    def generate_multi_batch(
        self, prompts: list[list[int]], num_samples: int = 1, **kwargs
    ) -> tuple[list[list[int]], list[list[int]]]:
        """generate_multi collected: (results, masks), len(prompts) *
        num_samples lists each, row p * num_samples + i for trajectory i of
        prompt p (the prompt followed by the generated tokens, masks 0 over
        the prompt)."""
        self._check_prompts(prompts)
        return self._collect(prompts, num_samples, kwargs, per_prompt=True)

    # -- shared machinery -------------------------------------------------------

    @staticmethod
    def _check_tokens(tokens) -> None:
        assert isinstance(tokens, list), "tokens must be a list of ints"
        assert len(tokens) > 0, "tokens must be non-empty"
        assert all(isinstance(t, int) for t in tokens), "tokens must be a list of ints"

    @classmethod
    def _check_prompts(cls, prompts) -> None:
        assert isinstance(prompts, list) and len(prompts) > 0, "prompts must be a non-empty list of token lists"
        for p in prompts:
            cls._check_tokens(p)
        assert len({len(p) for p in prompts}) == 1, "prompts must all have the same length"

    def _collect(self, prompts, num_samples, kwargs, per_prompt):
        unknown = set(kwargs) - {"max_tokens", "sampler", "seed", "force_schedule"}
        if unknown:
            raise TypeError(f"generate() got unexpected keyword arguments {sorted(unknown)}")
        rows = len(prompts) * num_samples
        columns, masks = [], []
        for column, mask in self._device_steps(
            prompts, num_samples, kwargs.get("max_tokens"), kwargs.get("sampler"), kwargs.get("seed", 42),
            kwargs.get("force_schedule"), per_prompt=per_prompt,
        ):
            columns.append(column)
            masks.append(mask)
        T, steps = len(prompts[0]), len(columns)
        # the mask of a step that samples or forces every row is known on the
        # host already; when every step is such a step all rows share one mask
        on_device = [s for s, m in enumerate(masks) if isinstance(m, torch.Tensor)]
        # about 2 * rows lists of Python ints are built here: with the garbage
        # collector running, a full collection triggered meanwhile walks every
        # list already built (measured: 100+ ms on a 6400-row call)
        gc_enabled = gc.isenabled()
        gc.disable()
        try:
            # the lists that need nothing from the device are built first,
            # while it still runs the steps enqueued above
            results = [prompts[r // num_samples].copy() for r in range(rows)]
            if not on_device:
                shared = [0] * T + [int(m) for m in masks]
                out_masks = [shared.copy() for _ in range(rows)]
            else:
                mask_np = np.empty((rows, steps), dtype=np.int64)
                for s, m in enumerate(masks):
                    if not isinstance(m, torch.Tensor):
                        mask_np[:, s] = m
                mask_np[:, on_device] = torch.stack([masks[s] for s in on_device], dim=1).cpu().numpy()
                zeros = [0] * T
                out_masks = [zeros + row for row in mask_np.tolist()]
            if gc_enabled:
                # the youngest generation's collection, which these lists
                # would trigger once the collector runs again, happens now:
                # while the device may still work, and over the rows before
                # the generated tokens lengthen them
                gc.collect(0)
            # the token columns reach the host in one copy
            if columns:
                for row, gen in zip(results, torch.stack(columns, dim=1).cpu().numpy().tolist()):
                    row += gen
        finally:
            if gc_enabled:
                gc.enable()
        return results, out_masks

    def _schedule(self, force_schedule, steps: int, n_prompts: int, num_samples: int, per_prompt: bool,
                  device) -> _Schedule | None:
        if force_schedule is None:
            return None
        rows = n_prompts * num_samples
        if not per_prompt or (len(force_schedule) > 0 and not isinstance(force_schedule[0], (list, tuple))
                              and not isinstance(force_schedule, np.ndarray)
                              and not isinstance(force_schedule, torch.Tensor)):
            assert len(force_schedule) >= steps, (
                f"force_schedule must cover all generation steps "
                f"(len={len(force_schedule)} < {steps})"
            )
            return _Schedule.shared_list(force_schedule, steps)
        if isinstance(force_schedule, (np.ndarray, torch.Tensor)):
            table = np.asarray(force_schedule.cpu() if isinstance(force_schedule, torch.Tensor) else force_schedule)
            assert table.ndim == 2 and table.shape[0] == rows, (
                f"a per-row force_schedule must be (rows={rows}, steps), got {table.shape}"
            )
        else:
            assert len(force_schedule) == n_prompts, (
                f"force_schedule must hold one schedule per prompt ({len(force_schedule)} != {n_prompts})"
            )
            width = min(len(s) for s in force_schedule)
            table = np.full((n_prompts, width), -1, dtype=np.int64)
            for p, s in enumerate(force_schedule):
                table[p] = [-1 if t is None else t for t in s[:width]]
            table = np.repeat(table, num_samples, axis=0)
        assert table.shape[1] >= steps, (
            f"force_schedule must cover all generation steps (len={table.shape[1]} < {steps})"
        )
        return _Schedule.table(table, steps, device)

    def _device_steps(
        self,
        prompts: list[list[int]],
        num_samples: int,
        max_tokens: int | None,
        sampler: Sampler | None,
        seed: int,
        force_schedule,
        per_prompt: bool,
    ) -> Generator[tuple[torch.Tensor, "int | torch.Tensor"], None, None]:
        """The generation loop with the token columns kept on the device:
        yields ((rows,) int64 column, mask) per step -- mask 1 / 0 for a step
        that samples / forces every row, a (rows,) int64 device tensor
        otherwise -- and feeds each column to the next decode forward without
        a host round trip."""
        T = len(prompts[0])
        S, N = len(prompts), num_samples
        rows = S * N
        steps = self._budget(T, max_tokens)
        if steps == 0:
            return

        model = self.model
        device = model.device_type
        schedule = self._schedule(force_schedule, steps, S, N, per_prompt, device)
        rng = torch.Generator(device=device)
        rng.manual_seed(seed)
        geometry = {
            "num_heads": model.n_head,
            "head_dim": model.n_embd // model.n_head,
            "num_layers": model.n_layer,
        }
        # the prefill's caller reads the last position's logits only
        prefill_kw = {"_last_only": True} if isinstance(model, GPT) else {}
        use_graph = self.use_graph and steps > 1 and torch.device(device).type == "cuda"
        key = self._graph_key(S, N, T, steps) if use_graph else None
        kept, self._kept = self._kept, None  # taken: a concurrent call builds its own
        reuse = kept is not None and kept[0] == key
        if kept is not None and not reuse:
            kept[2].close()
        ids = torch.tensor(prompts, dtype=torch.long, device=device)

        decode = None
        if N == 1:
            # one row per prompt: the prefill writes the decode cache itself
            if reuse:
                _, cache, decode = kept
                cache.reset()
            else:
                cache = KVCache(batch_size=S, seq_len=T + steps, **geometry)
            pos_dev, cache.pos_dev = cache.pos_dev, None  # a prefill, not the captured step
            try:
                logits, _ = model.forward(ids, kv_cache=cache, **prefill_kw)
            finally:
                cache.pos_dev = pos_dev
            logits = logits[:, -1, :]
        else:
            # 1) batched prefill of the prompts
            prompt_cache = KVCache(batch_size=S, seq_len=T, **geometry)
            logits, _ = model.forward(ids, kv_cache=prompt_cache, **prefill_kw)
            logits = logits[:, -1, :]
            logits = logits.expand(N, -1) if S == 1 else logits.repeat_interleave(N, dim=0)
            # 2) every row of a prompt starts from that prompt's cache, stored
            #    once as prefix pages (read once per decode step); a step
            #    captured by an earlier call with the same key replays into its
            #    own cache
            if reuse:
                _, cache, decode = kept
                cache._prefill_groups(prompt_cache, N, reuse=True)
            else:
                cache = KVCache(batch_size=rows, seq_len=T + steps, **geometry)
                cache._prefill_groups(prompt_cache, N)
            del prompt_cache
        if decode is not None:
            decode.rewind()
        elif use_graph:
            decode = _DecodeGraph(model, cache, rows, torch.device(device))

        try:
            for step in range(steps):
                kind = _SAMPLE if schedule is None else schedule.kinds[step]
                if kind == _FORCE_ALL:
                    if schedule.per_row is not None:
                        column = schedule.per_row[step]
                    else:
                        column = torch.full((rows,), schedule.shared[step], dtype=torch.long, device=logits.device)
                    mask = 0
                else:
                    if sampler is not None:
                        picked = sampler(logits, rng=rng)
                    else:
                        picked = draw_one(torch.softmax(logits, dim=-1), rng)
                    column = picked[:, 0]
                    mask = 1
                    if kind == _MIXED:
                        forced = schedule.per_row[step]
                        scheduled = forced >= 0
                        column = torch.where(scheduled, forced, column)
                        mask = (~scheduled).long()
                yield column, mask
                if step == steps - 1:
                    break  # the last column's logits would go unused

                # 3) one decode forward for the column just emitted
                step_ids = column.unsqueeze(1)
                if decode is not None:
                    logits = decode.step(step_ids)
                else:
                    logits, _ = model.forward(step_ids, kv_cache=cache)
                    logits = logits[:, -1, :]
        finally:
            if decode is not None:
                if cache.nbytes() <= _KEEP_GRAPH_BYTES:
                    self._kept = (key, cache, decode)
                else:
                    decode.close()


def _mask_list(mask, rows: int) -> list[int]:
    return mask.tolist() if isinstance(mask, torch.Tensor) else [mask] * rows
