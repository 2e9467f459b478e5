"""Forecasting API over the MI355X decode path (src/diff_gpt/diff_gpt.py:15-505).

DiffGPT wraps a GPT with the sigma-delta tokenizer's metadata (order of
derivative, domain of definition, Decimal mode).  A forecast encodes the
observed frame on the host (diff_gpt.encoder_decoder), prefills the prompt
once and decodes all requested trajectories together through the KV-cache
Engine -- whose broadcast cache makes every trajectory's attention read the
shared prompt once per series -- and decodes each trajectory's tokens back
to values.  Method names, arguments, defaults, assertion messages and
return shapes are the reference's.

Training (``train``, ``train_numa``) belongs to the reference's CPU/DDP
training stack and is not part of this inference build: those methods raise
and point at loading a trained state_dict instead.
"""

from __future__ import annotations

from typing import Callable

import numpy as np
import pandas as pd
import torch
import torch.nn.functional as F

from diff_gpt.encoder_decoder import decode, encode, np_to_decimal
from diff_gpt.model.engine import Engine
from diff_gpt.model.gpt import BaseGPT
from diff_gpt.sampler.sampler import Sampler

_NO_TRAINING = (
    "training is not part of the MI355X inference build: train with the reference "
    "package (fxeqxmulfx/diff-gpt) and load the state_dict here with DiffGPT.load / "
    "GPT.load_state_dict"
)


def _max_order(order: int | np.ndarray, n_columns: int, what: str) -> int:
    if isinstance(order, (int, np.integer)):
        return int(order)
    arr = np.asarray(order)
    assert arr.shape == (n_columns,), (
        f"order_of_derivative shape {arr.shape} must match {what} {n_columns}"
    )
    return int(arr.max())


class DiffGPT:
    __slots__ = (
        "model",
        "order_of_derivative",
        "domain_of_definition",
        "use_decimal",
    )

    def __init__(
        self,
        model: BaseGPT,
        order_of_derivative: int | np.ndarray,
        domain_of_definition: np.ndarray,
        use_decimal: bool,
    ) -> None:
        """
        `order_of_derivative`: scalar for uniform k across columns, or a
        length-F array for per-column k.
        """
        self.model = model
        self.order_of_derivative = order_of_derivative
        self.domain_of_definition = domain_of_definition
        self.use_decimal = use_decimal

    def train(self, *args, **kwargs) -> tuple[float, int]:
        raise NotImplementedError(_NO_TRAINING)

    @staticmethod
    def train_numa(
        model_factory: Callable[[int], BaseGPT],
        loader_factory: Callable,
        train_kwargs: dict | None = None,
        nodes: list[int] | None = None,
        checkpoint_path: str | None = None,
    ) -> tuple[float, int]:
        raise NotImplementedError(_NO_TRAINING)

    # ------------------------------------------------------------------ forecasting

    @torch.inference_mode()
    def predict(
        self,
        df: pd.DataFrame,
        max_new_points: int | None = None,
        future_covariates_df: pd.DataFrame | None = None,
        target_columns: "list[str] | list[int] | None" = None,
        sampler: Sampler | None = None,
    ) -> pd.DataFrame:
        """Forecast `max_new_points` rows after `df` (autoregressive), or, with
        `future_covariates_df` and `target_columns`, sample only the target
        columns while the others are teacher-forced from the known future
        (diff_gpt.py:127-177).  Returns the context rows followed by the
        forecast rows, with `df`'s columns."""
        if future_covariates_df is None:
            assert target_columns is None, (
                "target_columns is only meaningful with future_covariates_df"
            )
            assert max_new_points is not None, (
                "max_new_points is required when future_covariates_df is None"
            )
            future = self._generate_future_samples(
                df=df, max_new_points=max_new_points, sampler=sampler, num_samples=1
            )[0]
            full = np.concatenate([df.to_numpy(dtype=np.float64), future], axis=0)
            return pd.DataFrame(full, columns=df.columns)
        assert target_columns is not None and len(target_columns) > 0, (
            "target_columns must be non-empty when future_covariates_df is given"
        )
        pred_len = len(future_covariates_df)
        assert max_new_points is None or max_new_points == pred_len, (
            f"max_new_points ({max_new_points}) must equal "
            f"len(future_covariates_df) ({pred_len})"
        )
        return self._predict_teacher_forced(
            context_df=df,
            future_covariates_df=future_covariates_df,
            target_columns=target_columns,
            sampler=sampler,
        )

    def _encode_frame(self, frame: pd.DataFrame):
        values = frame.to_numpy(dtype=np.float64)
        if self.use_decimal:
            values = np_to_decimal(values)
        return encode(
            inp=values,
            vocab_size=self.model.vocab_size,
            domain_of_definition=self.domain_of_definition,
            order_of_derivative=self.order_of_derivative,
            use_decimal=self.use_decimal,
        )

    def _decode_tokens(self, start, scale, tokens: np.ndarray) -> np.ndarray:
        return decode(
            start=start,
            scale=scale,
            inp=tokens,
            vocab_size=self.model.vocab_size,
            order_of_derivative=self.order_of_derivative,
            use_decimal=self.use_decimal,
        )

    def _check_budget(self, df: pd.DataFrame, max_new_points: int) -> int:
        """The context checks of diff_gpt.py:209-214; returns the max order."""
        columns = df.shape[1]
        max_order = _max_order(self.order_of_derivative, columns, "columns")
        assert max_order <= df.shape[0], (
            f"max order {max_order} > context length {df.shape[0]}: "
            f"not enough history to compute the k-th derivative prefix"
        )
        total_positions = (df.shape[0] + max_new_points - max_order) * columns
        assert total_positions <= self.model.block_size, (
            f"prompt rows ({df.shape[0]}) + new points ({max_new_points}) with "
            f"{columns} columns (max_order={max_order}) require {total_positions} "
            f"context positions, but block_size is {self.model.block_size}"
        )
        return max_order

    def _generate_future_samples(
        self,
        df: pd.DataFrame,
        max_new_points: int,
        sampler: Sampler | None,
        num_samples: int,
    ) -> np.ndarray:
        """(num_samples, max_new_points, n_features) future rows
        (diff_gpt.py:179-253): one prompt prefill, all trajectories decoded
        together by Engine.generate_batch, each decoded on the host."""
        assert num_samples >= 1
        columns = df.shape[1]
        self._check_budget(df, max_new_points)
        start, scale, encoded = self._encode_frame(df)
        prompt = encoded.reshape(-1).astype(np.int64).tolist()
        results, _ = Engine(model=self.model).generate_batch(
            tokens=prompt,
            num_samples=num_samples,
            max_tokens=max_new_points * columns,
            sampler=sampler,
        )
        futures = np.empty((num_samples, max_new_points, columns), dtype=np.float64)
        lo, hi = df.shape[0], df.shape[0] + max_new_points
        for s, row in enumerate(results):
            values = self._decode_tokens(start, scale, np.asarray(row, dtype=np.int64).reshape(-1, columns))
            futures[s] = np.asarray(values[lo:hi], dtype=np.float64)
        return futures

    @torch.inference_mode()
    def predict_samples(
        self,
        df: pd.DataFrame,
        max_new_points: int,
        num_samples: int,
        sampler: Sampler | None = None,
    ) -> np.ndarray:
        """`num_samples` future trajectories, (num_samples, max_new_points,
        n_features) (diff_gpt.py:270-293)."""
        return self._generate_future_samples(
            df=df, max_new_points=max_new_points, sampler=sampler, num_samples=num_samples
        )

    @torch.inference_mode()
    def predict_samples_batch(
        self,
        dfs: "list[pd.DataFrame]",
        max_new_points: int,
        num_samples: int,
        sampler: Sampler | None = None,
        seed: int = 42,
    ) -> np.ndarray:
        """predict_samples for several series at once: (len(dfs),
        num_samples, max_new_points, n_features).  The frames must share their
        shape (the encoded prompts then share their length); their prompts are
        prefilled together and every trajectory of every series is decoded in
        one loop (Engine.generate_multi_batch), each series' prompt cache
        stored once and read once per step by its trajectories.  With a greedy
        sampler each series gets what predict_samples gives it; sampled
        trajectories draw from one generator for all series."""
        assert len(dfs) > 0, "dfs must be a non-empty list of frames"
        assert len({df.shape for df in dfs}) == 1, "all frames must have the same shape"
        columns = dfs[0].shape[1]
        self._check_budget(dfs[0], max_new_points)
        encoded = [self._encode_frame(df) for df in dfs]
        prompts = [e[2].reshape(-1).astype(np.int64).tolist() for e in encoded]
        results, _ = Engine(model=self.model).generate_multi_batch(
            prompts, num_samples=num_samples, max_tokens=max_new_points * columns, sampler=sampler, seed=seed,
        )
        out = np.empty((len(dfs), num_samples, max_new_points, columns), dtype=np.float64)
        lo, hi = dfs[0].shape[0], dfs[0].shape[0] + max_new_points
        for r, row in enumerate(results):
            start, scale, _ = encoded[r // num_samples]
            values = self._decode_tokens(start, scale, np.asarray(row, dtype=np.int64).reshape(-1, columns))
            out[r // num_samples, r % num_samples] = np.asarray(values[lo:hi], dtype=np.float64)
        return out

    @torch.inference_mode()
    def predict_batch(
        self,
        dfs: "list[pd.DataFrame]",
        future_covariates_dfs: "list[pd.DataFrame]",
        target_columns: "list[str] | list[int]",
        sampler: Sampler | None = None,
    ) -> "list[pd.DataFrame]":
        """The teacher-forced predict (diff_gpt.py:396-498) for several series
        at once: each series' covariate columns are forced from its own known
        future, so every series has a schedule of its own; all series decode
        in one loop (Engine.generate_multi_batch with per-prompt schedules).
        The frames and futures must share their shapes."""
        assert len(dfs) == len(future_covariates_dfs) and len(dfs) > 0, (
            "dfs and future_covariates_dfs must be non-empty lists of the same length"
        )
        assert len({df.shape for df in dfs}) == 1 and len({f.shape for f in future_covariates_dfs}) == 1, (
            "all frames (and all futures) must have the same shape"
        )
        plans = [self._forced_plan(df, fut, target_columns) for df, fut in zip(dfs, future_covariates_dfs)]
        n_prompt, total = plans[0][3], plans[0][4]
        results, _ = Engine(model=self.model).generate_multi_batch(
            [p[2][:n_prompt].tolist() for p in plans], num_samples=1, max_tokens=total - n_prompt,
            sampler=sampler, force_schedule=[p[5] for p in plans],
        )
        out = []
        for (start, scale, _, _, _, _, columns_list), row in zip(plans, results):
            n_features = len(columns_list)
            tokens = np.asarray(row, dtype=np.int64).reshape(-1, n_features)
            out.append(pd.DataFrame(self._decode_tokens(start, scale, tokens), columns=columns_list))
        return out

    @torch.inference_mode()
    def predict_quantiles(
        self,
        df: pd.DataFrame,
        max_new_points: int,
        quantiles: "list[float] | tuple[float, ...]" = (0.1, 0.5, 0.9),
        num_samples: int = 100,
        sampler: Sampler | None = None,
    ) -> dict[float, pd.DataFrame]:
        """Per-step empirical quantiles over `num_samples` trajectories
        (diff_gpt.py:365-394)."""
        for q in quantiles:
            assert 0.0 < q < 1.0, f"quantile {q} must be in (0, 1)"
        futures = self._generate_future_samples(
            df=df, max_new_points=max_new_points, sampler=sampler, num_samples=num_samples
        )
        return {
            float(q): pd.DataFrame(np.quantile(futures, q, axis=0), columns=df.columns)
            for q in quantiles
        }

    @torch.inference_mode()
    def anomaly_scores(self, df: pd.DataFrame) -> pd.DataFrame:
        """-log p(token_t | tokens_<t) per (row, column) from one causal
        forward over the encoded frame (diff_gpt.py:295-363); NaN where no
        token or no preceding context exists."""
        columns, n_rows = df.shape[1], df.shape[0]
        max_order = _max_order(self.order_of_derivative, columns, "columns")
        assert max_order <= n_rows, f"max order {max_order} > signal length {n_rows}"
        _, _, encoded = self._encode_frame(df)
        n_tok = encoded.size
        assert n_tok <= self.model.block_size, (
            f"signal has {n_tok} tokens but block_size is {self.model.block_size}; "
            f"chunk the input manually for longer sequences"
        )
        device = torch.device(self.model.device_type)
        tokens = torch.as_tensor(
            encoded.reshape(-1).astype(np.int64), dtype=torch.int64, device=device
        ).unsqueeze(0)
        was_training = self.model.training
        self.model.eval()
        logits, _ = self.model.forward(tokens)
        if was_training:
            self.model.train()
        logp = F.log_softmax(logits[0, :-1], dim=-1)  # row i predicts token i + 1
        nll = -logp.gather(-1, tokens[0, 1:].unsqueeze(-1)).squeeze(-1)
        flat = np.full(n_tok, np.nan, dtype=np.float64)
        flat[1:] = nll.detach().cpu().numpy().astype(np.float64)
        out = np.full((n_rows, columns), np.nan, dtype=np.float64)
        out[max_order:] = flat.reshape(encoded.shape[0], columns)
        return pd.DataFrame(out, columns=df.columns, index=df.index)

    def _forced_plan(
        self,
        context_df: pd.DataFrame,
        future_covariates_df: pd.DataFrame,
        target_columns: "list[str] | list[int]",
    ):
        """Encoding and force schedule of one teacher-forced forecast: (start,
        scale, tokens, n_prompt, total_tokens, schedule, columns)."""
        columns_list = list(context_df.columns)
        assert list(future_covariates_df.columns) == columns_list, (
            "context and future must have the same columns"
        )
        n_features = len(columns_list)
        targets: set[int] = set()
        for c in target_columns:
            if isinstance(c, str):
                assert c in columns_list, f"target column {c!r} not found in {columns_list}"
                targets.add(columns_list.index(c))
            else:
                targets.add(int(c))

        ctx_len, pred_len = len(context_df), len(future_covariates_df)
        max_order = _max_order(self.order_of_derivative, n_features, "n_features")
        assert max_order <= ctx_len, (
            f"max order {max_order} > context length {ctx_len}: "
            f"not enough history to compute the k-th derivative prefix"
        )
        total_tokens = (ctx_len + pred_len - max_order) * n_features
        assert total_tokens <= self.model.block_size, (
            f"ctx={ctx_len} pred={pred_len} cols={n_features} (max_order={max_order}) "
            f"need {total_tokens} tokens but block_size={self.model.block_size}"
        )

        # the future values of the target columns are unknown: encode zeros
        # there (their tokens are placeholders, replaced by sampling)
        frame = pd.concat([context_df, future_covariates_df], ignore_index=True).copy()
        for c in targets:
            frame.iloc[ctx_len:, c] = 0.0
        start, scale, encoded_full = self._encode_frame(frame)
        flat = encoded_full.reshape(-1).astype(np.int64).copy()

        n_prompt = (ctx_len - max_order) * n_features
        schedule: list[int | None] = [
            None if (p % n_features) in targets else int(flat[p])
            for p in range(n_prompt, total_tokens)
        ]
        return start, scale, flat, n_prompt, total_tokens, schedule, columns_list

    def _predict_teacher_forced(
        self,
        context_df: pd.DataFrame,
        future_covariates_df: pd.DataFrame,
        target_columns: "list[str] | list[int]",
        sampler: Sampler | None,
    ) -> pd.DataFrame:
        """Sample the target columns of the future rows, force the covariate
        columns from their known values (diff_gpt.py:396-498): the encoded
        context is the prompt and a force_schedule holds the covariate token
        of every future position that is not a target column."""
        start, scale, flat, n_prompt, total_tokens, schedule, columns_list = self._forced_plan(
            context_df, future_covariates_df, target_columns
        )
        results, _ = Engine(model=self.model).generate_batch(
            tokens=flat[:n_prompt].tolist(),
            num_samples=1,
            max_tokens=total_tokens - n_prompt,
            sampler=sampler,
            force_schedule=schedule,
        )
        tokens = np.asarray(results[0], dtype=np.int64).reshape(-1, len(columns_list))
        return pd.DataFrame(self._decode_tokens(start, scale, tokens), columns=columns_list)

    # ------------------------------------------------------------------ persistence

    def save(self, path: str = "diff-gpt.bin") -> None:
        torch.save(self.model.state_dict(), path)

    def load(self, path: str = "diff-gpt.bin") -> None:
        self.model.load_state_dict(torch.load(path, weights_only=True))
        self.model.eval()
