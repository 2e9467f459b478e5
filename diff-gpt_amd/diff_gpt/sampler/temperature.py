"""Temperature sampler (src/diff_gpt/sampler/temperature.py:6-26).

T == 0 is argmax (first maximum wins); otherwise one multinomial draw from
softmax(logits / T) with the caller's generator, on the logits' device.
The softmax and the Exp(1) variates stay torch's, so the RNG stream is
torch's; on the device the quotient and its argmax are one dg_draw_argmax
launch.
"""

import torch

from diff_gpt.sampler.sampler import Sampler


def draw_one(probs: torch.Tensor, rng: torch.Generator | None = None) -> torch.Tensor:
    """torch.multinomial(probs, num_samples=1, generator=rng): the same ids
    and the same use of the generator's stream, by torch's own single-draw
    algorithm -- an Exp(1) variate q per entry, then the first maximum of
    probs / q along the last dim -- without multinomial's validity checks
    (full-tensor min / max / sum reductions and device asserts, more than
    half of the sampling step's device time on a (6400, 256) batch).  Rows
    with inf, nan or negative entries, or summing to 0, which multinomial
    would reject, get an id here."""
    q = torch.empty_like(probs).exponential_(1, generator=rng)
    if probs.is_cuda:
        # the quotient and its first maximum in one launch (dg_draw_argmax)
        from diff_gpt import _native

        ids = torch.empty((*probs.shape[:-1], 1), dtype=torch.int64, device=probs.device)
        if _native.draw_argmax_(probs, q, ids):
            return ids
    return torch.argmax(probs / q, dim=-1, keepdim=True)


class TemperatureSampler(Sampler):
    """Sampler with Temperature"""

    __slots__ = "temperature"

    def __init__(self, temperature: float = 1.0) -> None:
        self.temperature = temperature

    def __call__(
        self, logits: torch.Tensor, rng: torch.Generator | None = None
    ) -> torch.Tensor:
        if self.temperature == 0:
            return torch.argmax(logits, dim=-1, keepdim=True)
        # x / 1 is x bit for bit: no division pass at temperature 1
        scaled = logits if self.temperature == 1 else logits / self.temperature
        return draw_one(torch.softmax(scaled, dim=-1), rng)
