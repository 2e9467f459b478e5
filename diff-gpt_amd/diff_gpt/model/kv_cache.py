"""Per-layer K/V cache in HBM (src/diff_gpt/model/kv_cache.py:4-116).

Physical layout is the reference's (L, 2, B, H, Tcap, D): for each (layer,
K|V, row, head) one contiguous page of Tcap*D elements, so a decode wavefront
streams one page front to back.  The observable behaviour is the reference's:
lazy allocation with the first inserted tensor's dtype/device, growth to
((t1 + 1024) + 1023) & ~1023 positions when an insert overflows, batch
broadcast on prefill, and ``pos`` advancing only after the last layer.

All data movement is done by libdgattn (dg_copy4d, or the fused
dg_rope_qknorm_append in MultiHeadAttention); only the bookkeeping is Python.
"""

import torch

from diff_gpt import _native


def _grown_capacity(t1: int) -> int:
    # kv_cache.py:92-96: what is needed plus 1024, rounded up to 1024
    return ((t1 + 1024) + 1023) & ~1023


def _pages(x: torch.Tensor, t: int) -> torch.Tensor:
    """(L,2,B,H,T,D) cache (or slice) -> 4-D (L*2, B, H, t*D) view of the first
    t positions of every page (positions and D are contiguous inside a page)."""
    L, two, B, H, _, D = x.shape
    st = x.stride()
    return x.as_strided((L * two, B, H, t * D), (st[1], st[2], st[3], 1))


class KVCache:
    """
    Works hand-in-hand with the GPT model to maintain the KV cache.
    Note that the .pos advances automatically after the last layer of the Transformer inserts.
    """

    __slots__ = (
        "kv_shape",
        "kv_cache",
        "pos",
        "shared_prefix",
        "pos_dev",
        "keys_normed",
    )

    def __init__(
        self,
        batch_size: int,
        num_heads: int,
        seq_len: int,
        head_dim: int,
        num_layers: int,
    ) -> None:
        self.kv_shape = (num_layers, 2, batch_size, num_heads, seq_len, head_dim)
        self.kv_cache = torch.zeros(0)
        self.pos = 0
        # (length, group) when rows come in groups of `group` consecutive rows
        # whose first `length` positions are identical (a batch-broadcast
        # prefill); decode attention then reads that prefix from the group's
        # first row only.  None otherwise.
        self.shared_prefix: tuple[int, int] | None = None
        # Device mirror of `pos` (one int32) while a captured decode step is in
        # use: the graph-replayable kernels read the position from it, and the
        # step advances both copies.  None in ordinary (eager) use.
        self.pos_dev: torch.Tensor | None = None
        # True while every key below pos was written by the model's attention
        # (RoPE + QK-norm, mha.py:44-48), i.e. every key row is RMS-normalised;
        # the prefill kernel then runs its softmax without a running maximum.
        # insert_kv with caller-supplied keys clears it.
        self.keys_normed = True

    def reset(self) -> None:
        self.pos = 0
        self.shared_prefix = None
        self.keys_normed = True

    def get_pos(self) -> int:
        return self.pos

    # -- prefill: batch-1 prompt cache -> num_samples rows (kv_cache.py:35-81) --
    def prefill(self, other: "KVCache") -> None:
        assert self.kv_cache.size(0) == 0, "Cannot prefill a non-empty KV cache"
        self._fill_from(other, reuse=False)

    def _refill(self, other: "KVCache") -> None:
        """prefill() into the tensor this cache already holds (same shape,
        dtype and device as a fresh prefill would allocate), so the pointers
        a captured decode step baked in stay valid."""
        assert self.kv_cache.size(0) != 0, "_refill needs an allocated cache"
        self._fill_from(other, reuse=True)

    def _fill_from(self, other: "KVCache", reuse: bool) -> None:
        assert other.kv_cache.size(0) != 0, "Cannot prefill with a None KV cache"
        sl, skv, sb, sh, st, sd = self.kv_shape
        ol, okv, ob, oh, ot, od = other.kv_shape
        assert sl == ol, f"Layer count mismatch: {sl} != {ol}"
        assert skv == okv, f"K/V dimension mismatch: {skv} != {okv}"
        assert sh == oh, f"Head count mismatch: {sh} != {oh}"
        assert sd == od, f"Head dim mismatch: {sd} != {od}"
        assert sb == ob or ob == 1, (
            f"Batch size mismatch: {sb} vs {ob} (other must be 1 or equal)"
        )
        assert st >= ot, f"Sequence length mismatch: {st} < {ot}"

        src = other.kv_cache
        _native.require_device("KVCache.prefill", src)
        if reuse:
            dst = self.kv_cache
            assert tuple(dst.shape) == tuple(self.kv_shape) and dst.dtype == src.dtype and dst.device == src.device, (
                "_refill: the held cache does not match the prompt cache"
            )
        else:
            self.kv_cache = torch.empty(self.kv_shape, dtype=src.dtype, device=src.device)
        n = other.pos
        if n > 0:
            dst4 = _pages(self.kv_cache, n)
            src4 = _pages(src, n)
            if ob == 1 and sb != 1:
                src4 = src4.expand(dst4.shape)  # batch broadcast: 0 stride on B
            _native.ops().copy4d(src4, dst4)
        self.pos = n
        self.shared_prefix = (n, sb) if (ob == 1 and sb > 1 and n > 0) else None
        self.keys_normed = other.keys_normed

    # -- capacity management shared by insert_kv and the fused MHA path --
    def ensure_window(
        self, T_add: int, dtype: torch.dtype, device: torch.device
    ) -> tuple[int, int]:
        """Make room for T_add more positions at ``pos``; returns (t0, t1)."""
        if self.kv_cache.size(0) == 0:
            _native.require_device_type("KVCache", device)
            self.kv_cache = torch.empty(self.kv_shape, dtype=dtype, device=device)
        t0, t1 = self.pos, self.pos + T_add
        if self.shared_prefix is not None and t0 < self.shared_prefix[0]:
            # rows diverge from position t0 on: only the part before it stays shared
            self.shared_prefix = (t0, self.shared_prefix[1]) if t0 > 0 else None
        cap = self.kv_cache.size(4)
        if t1 > cap:
            new_cap = _grown_capacity(t1)
            old = self.kv_cache
            shape = list(old.shape)
            shape[4] = new_cap
            grown = torch.empty(shape, dtype=old.dtype, device=old.device)
            if cap > 0:
                _native.ops().copy4d(_pages(old, cap), _pages(grown, cap))
            self.kv_cache = grown
            self.kv_shape = tuple(grown.shape)
        return t0, t1

    def layer_views(self, layer_idx: int, t1: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(B,H,t1,D) views of layer ``layer_idx``'s keys and values."""
        return (
            self.kv_cache[layer_idx, 0, :, :, :t1, :],
            self.kv_cache[layer_idx, 1, :, :, :t1, :],
        )

    def advance(self, layer_idx: int, t1: int) -> None:
        """pos moves once the last layer has written its window (kv_cache.py:113-115)."""
        if layer_idx == self.kv_cache.size(0) - 1:
            self.pos = t1

    # -- reference entry point: copy ready-made k/v (B,H,T,D) into the cache --
    def insert_kv(
        self, layer_idx: int, k: torch.Tensor, v: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        _native.require_device("KVCache.insert_kv", k, v)
        _native.require_inference("KVCache.insert_kv", k, v)
        B, H, T_add, D = k.size()
        t0, t1 = self.ensure_window(T_add, k.dtype, k.device)
        cache = self.kv_cache
        if k.dtype != cache.dtype:
            k = k.to(cache.dtype)
        if v.dtype != cache.dtype:
            v = v.to(cache.dtype)
        _native.ops().copy4d(k, cache[layer_idx, 0, :, :, t0:t1, :])
        _native.ops().copy4d(v, cache[layer_idx, 1, :, :, t0:t1, :])
        self.keys_normed = False  # keys from the caller: no norm to rely on
        key_view, value_view = self.layer_views(layer_idx, t1)
        self.advance(layer_idx, t1)
        return key_view, value_view
