"""Transformer block with Block Attention Residuals (src/diff_gpt/model/block.py:10-107).

Each sub-layer (attention, MLP) reads a per-token softmax mixture over the
committed block states plus the running partial sum, weighted by a learned
pseudo-query; a block boundary every ``layers_per_block`` layers commits the
partial sum.  In Block.forward the mixture and the RMSNorm after it are one
dg_attn_res_norm launch, the clamped SwiGLU of the MLP one dg_swiglu launch,
and the attention sub-layer is the HIP path of MultiHeadAttention.  At
n_embd 64 or 128 everything after the attention -- gate, c_proj, the partial
sum, the MLP's mixture and norm, the FFN and the residual -- is one
dg_block_out launch instead of six.
``block_attn_res`` keeps the reference's torch formulation for direct callers.
"""

import torch
import torch.nn.functional as F
from torch import nn

from diff_gpt import _native
from diff_gpt.model.feed_forward import FeedForward
from diff_gpt.model.kv_cache import KVCache
from diff_gpt.model.mha import MultiHeadAttention
from diff_gpt.model.rms_norm import rms_norm

# dg_attn_res_norm takes at most this many sources of at most this width
ATTN_RES_MAX_SOURCES = 32
ATTN_RES_MAX_WIDTH = 2048

def block_attn_res(
    blocks: tuple[torch.Tensor, ...],
    partial_block: torch.Tensor,
    proj: nn.Linear,
) -> torch.Tensor:
    """softmax_n(rms_norm(V_n) . w) weighted sum of V_n over V = (*blocks, partial),
    per token (block.py:10-44).  With a single committed block that *is* the
    partial sum (layer 0) the mixture is that tensor itself."""
    if len(blocks) == 1 and partial_block is blocks[0]:
        return partial_block
    V = torch.stack((*blocks, partial_block), dim=0)  # (N+1, B, T, C)
    scores = rms_norm(V).matmul(proj.weight.view(-1))  # (N+1, B, T)
    weights = scores.softmax(dim=0).unsqueeze(-1)
    return (weights * V).sum(dim=0)


def attn_res_norm(
    blocks: tuple[torch.Tensor, ...],
    partial_block: torch.Tensor,
    proj: nn.Linear,
) -> torch.Tensor:
    """rms_norm(block_attn_res(blocks, partial_block, proj)) in one launch
    (dg_attn_res_norm), with block_attn_res's single-block short cut."""
    if len(blocks) == 1 and partial_block is blocks[0]:
        return rms_norm(partial_block)
    if len(blocks) + 1 > ATTN_RES_MAX_SOURCES or partial_block.size(-1) > ATTN_RES_MAX_WIDTH:
        # beyond the fused kernel's limits: the mixture as device torch ops,
        # then the RMSNorm kernel
        return rms_norm(block_attn_res(blocks, partial_block, proj))
    return _native.ops().attn_res_norm([*blocks, partial_block], proj.weight)


class Block(nn.Module):
    def __init__(
        self,
        n_embd: int,
        n_head: int,
        swiglu_alpha: float,
        swiglu_limit: float,
        layer_idx: int,
        layers_per_block: int = 1,
    ) -> None:
        super().__init__()
        assert layers_per_block >= 1
        self.layer_idx = layer_idx
        self.layers_per_block = layers_per_block
        self.sa = MultiHeadAttention(n_embd=n_embd, n_head=n_head, layer_idx=layer_idx)
        self.ffwd = FeedForward(
            n_embd=n_embd, swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit
        )
        # one (1, C) pseudo-query per sub-layer
        self.attn_res_proj = nn.Linear(n_embd, 1, bias=False)
        self.mlp_res_proj = nn.Linear(n_embd, 1, bias=False)

    def _at_boundary(self) -> bool:
        return (self.layer_idx + 1) % self.layers_per_block == 0

    def forward(
        self,
        blocks: tuple[torch.Tensor, ...],
        partial_block: torch.Tensor,
        freqs_cis: torch.Tensor,
        kv_cache: KVCache | None,
        *,
        _last_only: bool = False,
        _xn: torch.Tensor | None = None,
        _xn_out: torch.Tensor | None = None,
    ) -> tuple[tuple[torch.Tensor, ...], torch.Tensor]:
        """block.py:87-107.  With _last_only the attention still runs over
        every position (its keys and values go to the cache), and the rest of
        the layer only for the last one: the outputs are that position's
        (B, 1, C) rows, for a last layer whose other rows only the logits of
        their own positions would read.  _xn, when given, is the attention
        sub-layer's input attn_res_norm(blocks, partial_block) computed by the
        caller (layer 0's, from the embedding launch).  _xn_out, when given
        (shaped as the returned partial sum), receives rms_norm of it: the
        head's input after the last layer, from the same launch when
        dg_block_out takes the layer."""
        _native.require_device("Block", partial_block)
        xn = attn_res_norm(blocks, partial_block, self.attn_res_proj) if _xn is None else _xn
        committed = self._at_boundary()
        partial_in = partial_block
        if committed:
            blocks = (*blocks, partial_block)
        sa = self.sa
        qkvg = F.linear(xn, sa._projection_weight())
        y = sa._attend(qkvg, freqs_cis, kv_cache)
        g = sa._gate_logits(qkvg)
        if _last_only:
            y, g, partial_in = y[:, -1:], g[:, -1:], partial_in[:, -1:]
            blocks = tuple(b[:, -1:] for b in blocks)
        up, swiglu, down = self.ffwd.net
        if len(blocks) + 1 <= ATTN_RES_MAX_SOURCES:
            # gate, c_proj, the partial sum, the MLP's mixture and norm, the FFN
            # and the residual in one launch (n_embd 64 or 128)
            out = torch.empty_like(partial_in)
            if _native.block_out_(y, g, sa.c_proj.weight, None if committed else partial_in, list(blocks),
                                  self.mlp_res_proj.weight, up.weight, down.weight, swiglu.alpha, swiglu.limit,
                                  out, _xn_out):
                return blocks, out
        _native.ops().gate_(y, g)  # y * sigmoid(g), mha.py:84
        attn_out = sa.c_proj(y)
        partial_block = attn_out if committed else partial_in + attn_out
        out = self._mlp(blocks, partial_block)
        if _xn_out is not None:
            _native.rms_norm_(out, _xn_out)
        return blocks, out

    def _mlp(self, blocks: tuple[torch.Tensor, ...], partial_block: torch.Tensor) -> torch.Tensor:
        xn = attn_res_norm(blocks, partial_block, self.mlp_res_proj)
        up, swiglu, down = self.ffwd.net
        hidden = _native.ops().swiglu(F.linear(xn, up.weight), swiglu.alpha, swiglu.limit)
        return partial_block + F.linear(hidden, down.weight)
