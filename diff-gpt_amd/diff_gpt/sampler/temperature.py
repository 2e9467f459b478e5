"""Temperature sampler (src/diff_gpt/sampler/temperature.py:6-26).

T == 0 is argmax (first maximum wins); otherwise one multinomial draw from
softmax(logits / T) with the caller's generator, on the logits' device.
Kept on torch so the RNG stream is torch's.
"""

import torch

from diff_gpt.sampler.sampler import Sampler


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
        probs = torch.softmax(logits / self.temperature, dim=-1)
        return torch.multinomial(probs, num_samples=1, generator=rng)
