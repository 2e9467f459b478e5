"""Parameter-free RMSNorm over the last axis (src/diff_gpt/model/rms_norm.py:5-7).

F.rms_norm with eps=None: y = x * rsqrt(mean(x^2) + FLT_EPSILON), computed in
fp32 and rounded once to x's dtype.  Runs as the HIP kernel dg_rms_norm.
"""

import torch

from diff_gpt import _native


def rms_norm(x: torch.Tensor) -> torch.Tensor:
    _native.require_device("rms_norm", x)
    _native.require_inference("rms_norm", x)
    return _native.ops().rms_norm(x)
