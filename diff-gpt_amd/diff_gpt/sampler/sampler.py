"""Token sampler interface (src/diff_gpt/sampler/sampler.py:4-11)."""

import torch


class Sampler:
    """Base class for token samplers."""

    def __call__(
        self, logits: torch.Tensor, rng: torch.Generator | None = None
    ) -> torch.Tensor:
        """Sample from logits of shape `[..., n_tokens]`; returns `[..., 1]` ids."""
        raise NotImplementedError()
