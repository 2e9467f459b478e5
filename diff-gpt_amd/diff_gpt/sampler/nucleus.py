"""Nucleus (top-p) sampler (src/diff_gpt/sampler/nucleus.py:7-40).

Keeps the smallest prefix of tokens, in descending probability, whose mass
reaches p (the token that crosses p is kept, the top token always is), sets
every other logit to -inf and hands the result to the inner sampler.
"""

import torch

from diff_gpt.sampler.sampler import Sampler


class NucleusSampler(Sampler):
    """Nucleus Sampler"""

    __slots__ = (
        "p",
        "sampler",
    )

    def __init__(self, p: float, sampler: Sampler) -> None:
        self.p = p
        self.sampler = sampler

    def __call__(
        self, logits: torch.Tensor, rng: torch.Generator | None = None
    ) -> torch.Tensor:
        probs = torch.softmax(logits, dim=-1)
        sorted_probs, order = torch.sort(probs, dim=-1, descending=True)
        # rank r is kept iff the cumulative mass through rank r-1 is < p;
        # rank 0 is always kept
        keep_sorted = torch.ones_like(sorted_probs, dtype=torch.bool)
        keep_sorted[..., 1:] = torch.cumsum(sorted_probs, dim=-1)[..., :-1] < self.p
        keep = torch.zeros_like(keep_sorted).scatter_(-1, order, keep_sorted)
        masked = logits.masked_fill(~keep, float("-inf"))
        return self.sampler(masked, rng=rng)
