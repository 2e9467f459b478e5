"""Gated multi-head self-attention (src/diff_gpt/model/mha.py:10-86).

Projections, the sigmoid gate and the output projection stay on hipBLASLt via
nn.Linear.  Everything between the projections and the gate runs in libdgattn:

  one dg_rope_qknorm_append launch  -- RoPE on q and k, QK-norm, and the K/V
                                       append into the cache page at ``pos``
                                       (mha.py:44-56, kv_cache.py:108-109)
  one dg_attention launch           -- causal prefill / single-token decode /
                                       chunked prefill (mha.py:61-81), written
                                       straight into the (B,T,H*D) layout that
                                       mha.py:83 re-assembles.
"""

import math

import torch
from torch import nn

from diff_gpt import _native
from diff_gpt.model.kv_cache import KVCache


class MultiHeadAttention(nn.Module):
    def __init__(
        self,
        n_embd: int,
        n_head: int,
        layer_idx: int,
    ) -> None:
        super().__init__()
        assert n_embd % n_head == 0
        # RoPE rotates (even, odd) pairs, so head_dim must be even.
        assert (n_embd // n_head) % 2 == 0
        self.n_embd = n_embd
        self.n_head = n_head
        self.layer_idx = layer_idx
        self.head_dim = self.n_embd // self.n_head
        inner = self.n_head * self.head_dim
        # creation order fixes the parameter initialisation order (seeded RNG)
        self.c_q = nn.Linear(self.n_embd, inner, bias=False)
        self.c_k = nn.Linear(self.n_embd, inner, bias=False)
        self.c_v = nn.Linear(self.n_embd, inner, bias=False)
        self.c_g = nn.Linear(self.n_embd, self.n_embd, bias=False)
        self.c_proj = nn.Linear(self.n_embd, self.n_embd, bias=False)

    def forward(
        self,
        x: torch.Tensor,
        freqs_cis: torch.Tensor,
        kv_cache: KVCache | None,
    ) -> torch.Tensor:
        _native.require_device("MultiHeadAttention", x)
        _native.require_inference("MultiHeadAttention", x, self.c_q.weight)
        B, T, _ = x.size()
        H, D = self.n_head, self.head_dim
        ops = _native.ops()

        q = self.c_q(x).view(B, T, H, D)
        k = self.c_k(x).view(B, T, H, D)
        v = self.c_v(x).view(B, T, H, D)
        g = self.c_g(x)

        q_rot = torch.empty((B, T, H, D), dtype=q.dtype, device=q.device)
        if kv_cache is not None and kv_cache.pos_dev is not None:
            return self._decode_step_at(q, k, v, g, q_rot, freqs_cis, kv_cache)
        if kv_cache is None:
            # no cache: normalised keys go to a scratch tensor, values are read
            # in place from the projection output
            k_rot = torch.empty_like(q_rot)
            ops.rope_qknorm_append(q, k, None, freqs_cis, q_rot, k_rot, None, True)
            keys, values = k_rot, v
        else:
            t0, t1 = kv_cache.ensure_window(T, k.dtype, k.device)
            cache = kv_cache.kv_cache
            if cache.dtype != k.dtype:
                raise TypeError(
                    f"KV cache holds {cache.dtype} but the layer computes in {k.dtype}"
                )
            # (B,H,T,D) cache pages seen as (B,T,H,D) views
            k_dst = cache[self.layer_idx, 0, :, :, t0:t1, :].transpose(1, 2)
            v_dst = cache[self.layer_idx, 1, :, :, t0:t1, :].transpose(1, 2)
            ops.rope_qknorm_append(q, k, v, freqs_cis, q_rot, k_dst, v_dst, True)
            k_all, v_all = kv_cache.layer_views(self.layer_idx, t1)
            keys, values = k_all.transpose(1, 2), v_all.transpose(1, 2)
            kv_cache.advance(self.layer_idx, t1)
            shared = kv_cache.shared_prefix

        # SDPA default scale 1/sqrt(head_dim); the mask follows from Tq vs Tk.
        # A broadcast prefix (KVCache.prefill) is read once per row group.
        prefix_len, group = (0, 1) if kv_cache is None or shared is None else shared
        y = ops.attention(q_rot, keys, values, 1.0 / math.sqrt(D), prefix_len, group)
        y = y.view(B, T, H * D)
        y = y * torch.sigmoid(g)
        return self.c_proj(y)

    def _decode_step_at(self, q, k, v, g, q_rot, freqs_table, kv_cache: KVCache) -> torch.Tensor:
        """One decode token per row with the position read on the device
        (kv_cache.pos_dev): the same arithmetic as forward(), in the launch form
        a HIP graph can replay at every position.  freqs_table is the model's
        whole (Tmax, D/2, 2) table."""
        B, T, H, D = q.shape
        assert T == 1, "a captured decode step takes one token per row"
        t0, t1 = kv_cache.ensure_window(1, k.dtype, k.device)
        cache = kv_cache.kv_cache
        assert cache.size(4) >= t1, "the cache must not grow inside a captured decode step"
        k_cache = cache[self.layer_idx, 0].transpose(1, 2)  # (B, Tcap, H, D) at position 0
        v_cache = cache[self.layer_idx, 1].transpose(1, 2)
        _native.rope_qknorm_append_at_(q, k, v, freqs_table, q_rot, k_cache, v_cache, kv_cache.pos_dev, True)
        kv_cache.advance(self.layer_idx, t1)
        prefix_len, group = (0, 1) if kv_cache.shared_prefix is None else kv_cache.shared_prefix
        y = torch.empty_like(q_rot)
        _native.decode_attention_at_(q_rot, k_cache, v_cache, y, 1.0 / math.sqrt(D), kv_cache.pos_dev,
                                     prefix_len, group)
        y = y.view(B, T, H * D) * torch.sigmoid(g)
        return self.c_proj(y)
