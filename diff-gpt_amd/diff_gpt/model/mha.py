"""Gated multi-head self-attention (src/diff_gpt/model/mha.py:10-86).

The q, k, v and g projections are one GEMM (hipBLASLt) against one storage
that the four weight parameters are row views of; q, k, v and g are column
slices of its output, which the kernels read through strides.
The sigmoid gate is one dg_gate launch and the output projection a GEMM.
Everything between the projections and the gate runs in libdgattn:

  one dg_rope_qknorm_append launch  -- RoPE on q and k, QK-norm, and the K/V
                                       append into the cache page at ``pos``
                                       (mha.py:44-56, kv_cache.py:108-109)
  one dg_attention launch           -- causal prefill / single-token decode /
                                       chunked prefill (mha.py:61-81), written
                                       straight into the (B,T,H*D) layout that
                                       mha.py:83 re-assembles.

A prefill that the MFMA kernel takes (bf16/fp16, head_dim 64 or 128, at
least 16 tokens) leaves q to the attention launch instead: dg_prefill_rope
rotates and normalises the query rows as it loads them, with the bits the
first launch would have stored.

A decode step over a KV cache (one new token per row) makes one
dg_decode_step call instead: the same RoPE, QK-norm and append, and the
attention over the cache including the new token, in one launch where the
rows share a broadcast prefix (two launches otherwise).

Block.forward runs the projection itself and may run the gate and c_proj
too (dg_block_out, fused with the MLP after them); it then calls _attend, the
part between, directly.
"""

import math

import torch
import torch.nn.functional as F
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
        # the reference's SDPA takes any even head_dim; the HIP kernels have
        # limits, checked here rather than at the first launch
        if not _native.head_dim_supported(self.head_dim):
            raise ValueError(
                f"head_dim {self.head_dim} (n_embd {n_embd} / n_head {n_head}) is beyond the HIP attention "
                f"kernels, which take even head dims up to {_native.MAX_HEAD_DIM}"
            )
        inner = self.n_head * self.head_dim
        # creation order fixes the parameter initialisation order (seeded RNG)
        self.c_q = nn.Linear(self.n_embd, inner, bias=False)
        self.c_k = nn.Linear(self.n_embd, inner, bias=False)
        self.c_v = nn.Linear(self.n_embd, inner, bias=False)
        self.c_g = nn.Linear(self.n_embd, self.n_embd, bias=False)
        self.c_proj = nn.Linear(self.n_embd, self.n_embd, bias=False)
        self._qkvg: torch.Tensor | None = None
        self._tie_projections()

    def _weights4(self) -> tuple[torch.Tensor, ...]:
        return (self.c_q.weight, self.c_k.weight, self.c_v.weight, self.c_g.weight)

    def _tie_projections(self) -> None:
        """Place the c_q, c_k, c_v and c_g weights in one (3*inner + C, C)
        storage, rows in that order, and make each parameter a view of its
        rows.  The four projections are then one GEMM against that storage,
        and any update of a parameter -- in place, through .data, or by
        load_state_dict -- is an update of the storage itself: there is no
        second copy that could go stale."""
        ws = self._weights4()
        fused = torch.cat([w.detach() for w in ws], dim=0)
        row = 0
        for w in ws:
            n = w.size(0)
            w.data = fused[row : row + n]
            row += n
        self._qkvg = fused

    def _is_tied(self) -> bool:
        fused = self._qkvg
        if fused is None:
            return False
        row_bytes = fused.stride(0) * fused.element_size()
        row = 0
        for w in self._weights4():
            if (
                w.dtype != fused.dtype
                or w.device != fused.device
                or w.stride() != fused.stride()
                or w.data_ptr() != fused.data_ptr() + row * row_bytes
            ):
                return False
            row += w.size(0)
        return row == fused.size(0)

    def _apply(self, fn, recurse=True):
        # .to() / .cuda() / .bfloat16() convert each parameter on its own;
        # gather the converted weights into one storage again
        super()._apply(fn, recurse)
        self._tie_projections()
        return self

    def _projection_weight(self) -> torch.Tensor:
        """The (3*inner + C, C) storage that c_q, c_k, c_v and c_g view; re-tied
        first if a parameter was replaced by another tensor."""
        if not self._is_tied():
            self._tie_projections()
        return self._qkvg

    def forward(
        self,
        x: torch.Tensor,
        freqs_cis: torch.Tensor,
        kv_cache: KVCache | None,
    ) -> torch.Tensor:
        _native.require_device("MultiHeadAttention", x)
        _native.require_inference("MultiHeadAttention", x, self.c_q.weight)
        qkvg = F.linear(x, self._projection_weight())  # (B, T, 3*inner + C)
        y = self._attend(qkvg, freqs_cis, kv_cache)
        ops = _native.ops()
        ops.gate_(y, self._gate_logits(qkvg))  # y * sigmoid(g)
        return self.c_proj(y)

    def _gate_logits(self, qkvg: torch.Tensor) -> torch.Tensor:
        return qkvg[..., 3 * self.n_head * self.head_dim :]

    def _attend(self, qkvg: torch.Tensor, freqs_cis: torch.Tensor, kv_cache: KVCache | None) -> torch.Tensor:
        """mha.py:44-83 on the projections qkvg (B, T, 3*inner + C), whose
        column slices are q, k, v and the gate logits: RoPE, QK-norm, the
        cache append and the attention; returns y (B, T, inner) before the
        gate."""
        B, T, _ = qkvg.size()
        H, D = self.n_head, self.head_dim
        ops = _native.ops()
        inner = H * D
        q = qkvg[..., :inner].view(B, T, H, D)
        k = qkvg[..., inner : 2 * inner].view(B, T, H, D)
        v = qkvg[..., 2 * inner : 3 * inner].view(B, T, H, D)

        if kv_cache is not None and T == 1:
            return self._decode_step(q, k, v, freqs_cis, kv_cache)
        assert kv_cache is None or kv_cache.pos_dev is None, "a captured decode step takes one token per row"
        # Prefills the MFMA kernel takes rotate and normalise q as they load it
        # (dg_prefill_rope); the first launch then handles k and v only.
        fuse_q = T >= 16 and D in (64, 128) and q.dtype in (torch.bfloat16, torch.float16, torch.float32)
        q_rot = None if fuse_q else torch.empty((B, T, H, D), dtype=q.dtype, device=q.device)
        q_in = None if fuse_q else q
        if kv_cache is None:
            # no cache: normalised keys go to a scratch tensor, values are read
            # in place from the projection output
            k_rot = torch.empty((B, T, H, D), dtype=q.dtype, device=q.device)
            ops.rope_qknorm_append(q_in, k, None, freqs_cis, q_rot, k_rot, None, True)
            keys, values = k_rot, v
            keys_normed = True
        else:
            t0, t1 = kv_cache.ensure_window(T, k.dtype, k.device)
            cache = kv_cache._tensor()
            if cache.dtype != k.dtype:
                raise TypeError(
                    f"KV cache holds {cache.dtype} but the layer computes in {k.dtype}"
                )
            # (B,H,T,D) cache pages seen as (B,T,H,D) views
            k_dst = cache[self.layer_idx, 0, :, :, t0:t1, :].transpose(1, 2)
            v_dst = cache[self.layer_idx, 1, :, :, t0:t1, :].transpose(1, 2)
            ops.rope_qknorm_append(q_in, k, v, freqs_cis, q_rot, k_dst, v_dst, True)
            k_all, v_all = kv_cache.layer_views(self.layer_idx, t1)
            keys, values = k_all.transpose(1, 2), v_all.transpose(1, 2)
            kv_cache.advance(self.layer_idx, t1)
            shared = kv_cache.shared_prefix
            keys_normed = kv_cache.keys_normed

        # SDPA default scale 1/sqrt(head_dim); the mask follows from Tq vs Tk.
        # A broadcast prefix (KVCache.prefill) is read once per row group.
        prefix_len, group = (0, 1) if kv_cache is None or shared is None else shared
        scale = 1.0 / math.sqrt(D)
        y = None
        if fuse_q:
            y = torch.empty((B, T, H, D), dtype=q.dtype, device=q.device)
            # every key normalised (mha.py:48): the kernel's bounded softmax
            if not _native.prefill_rope_(q, freqs_cis, keys, values, y, scale, True, keys_normed):
                # a layout the fused kernel does not take (alignment): rotate q apart
                q_rot = torch.empty_like(y)
                ops.rope_qknorm_append(q, None, None, freqs_cis, q_rot, None, None, True)
                y = None
        if y is None:
            y = ops.attention(q_rot, keys, values, scale, prefix_len, group)
        return y.view(B, T, H * D)

    def _decode_step(self, q, k, v, freqs, kv_cache: KVCache) -> torch.Tensor:
        """One new token per row over the KV cache (mha.py:44-68 with T = 1):
        dg_decode_step appends k, v at the cache position and attends over it.
        With kv_cache.pos_dev set the position is read on the device (the
        launch form a HIP graph replays at every position) and freqs is the
        model's whole (Tmax, D/2, 2) table; otherwise freqs is the row of the
        current position.  Returns y (B, 1, inner) before the gate."""
        B, T, H, D = q.shape
        cap = kv_cache.kv_shape[4]
        t0, t1 = kv_cache.ensure_window(1, k.dtype, k.device)
        # the rows' pages (B, positions, H, D) from position own_start, and the
        # broadcast prefix (KVCache.prefill), read once per row group
        k_cache, v_cache, prefix = kv_cache.decode_views(self.layer_idx)
        if k_cache.dtype != k.dtype:
            raise TypeError(f"KV cache holds {k_cache.dtype} but the layer computes in {k.dtype}")
        if kv_cache.pos_dev is not None:
            assert cap >= t1, "the cache must not grow inside a captured decode step"
            pos = kv_cache.pos_dev
        else:
            pos = t0
        y = torch.empty_like(q)
        _native.decode_step_(q, k, v, freqs, k_cache, v_cache, y, 1.0 / math.sqrt(D), pos, prefix=prefix)
        kv_cache.advance(self.layer_idx, t1)
        return y.view(B, T, H * D)
