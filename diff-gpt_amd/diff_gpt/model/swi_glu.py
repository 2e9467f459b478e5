"""Clamped SwiGLU with +1 on the linear half (src/diff_gpt/model/swi_glu.py:5-19).

Model plumbing outside the attention hot path: plain torch elementwise ops.
The input's last axis interleaves (gate, linear) as x[..., 0::2], x[..., 1::2].
"""

import torch
from torch import nn


class SwiGLU(nn.Module):
    def __init__(self, alpha: float, limit: float):
        super().__init__()
        self.alpha = alpha
        self.limit = limit

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate = x[..., 0::2].clamp(max=self.limit)
        lin = x[..., 1::2].clamp(min=-self.limit, max=self.limit)
        return gate * torch.sigmoid(self.alpha * gate) * (lin + 1)
