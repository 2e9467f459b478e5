"""Rotary embedding: the (cos, sin) table and its application.

Reference: src/diff_gpt/model/rope.py:4-44.  The table is built once, on the
host, at model construction (gpt.py:131-135) and then lives on the device as a
module buffer; the rotation itself is the HIP kernel dg_rope_qknorm_append
(without the norm), which reads that same buffer.
"""

import torch

from diff_gpt import _native


def apply_rotary_emb(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    """Rotate interleaved pairs (x[2j], x[2j+1]) of the last axis by the
    (cos, sin) pairs of ``freqs_cis`` (shape (..., D/2, 2), broadcast against
    x's leading dims); fp32 arithmetic, result in x's dtype (rope.py:4-27)."""
    _native.require_device("apply_rotary_emb", x, freqs_cis)
    _native.require_inference("apply_rotary_emb", x, freqs_cis)
    if x.size(-1) % 2 != 0:
        raise ValueError(f"apply_rotary_emb: last dim must be even, got {x.size(-1)}")
    return _native.ops().rope(x, freqs_cis)


def precompute_freqs_cis(dim: int, end: int, theta: float) -> torch.Tensor:
    """(end, dim/2, 2) fp32 table: row m, pair j = (cos m*w_j, sin m*w_j) with
    w_j = theta**(-2j/dim) (rope.py:30-44).  Built with torch on the host so
    the values are the ones the reference holds in its buffer."""
    half = dim // 2
    exponent = torch.arange(0, dim, 2, dtype=torch.float32)[:half] / dim
    inv_freq = 1.0 / (theta**exponent)
    pos = torch.arange(end, dtype=torch.float32)
    angle = pos[:, None] * inv_freq[None, :]
    return torch.stack((angle.cos(), angle.sin()), dim=-1)
