"""Per-layer K/V cache in HBM (src/diff_gpt/model/kv_cache.py:4-116).

Physical layout is the reference's (L, 2, B, H, Tcap, D): for each (layer,
K|V, row, head) one contiguous page of Tcap*D elements, so a decode wavefront
streams one page front to back.  The observable behaviour is the reference's:
lazy allocation with the first inserted tensor's dtype/device, growth to
((t1 + 1024) + 1023) & ~1023 positions when an insert overflows, batch
broadcast on prefill, and ``pos`` advancing only after the last layer.

Shared prefix stored once.  KVCache.prefill from a batch-1 cache (the
reference broadcasts it into every row, kv_cache.py:77-79) stores the prefix
once, as (L, 2, G, H, P, D) prefix pages, and gives each row pages for its own
positions only, (L, 2, B, H, Tcap - P, D).  Decode attention reads each
group's prefix from its pages (the kernels take it as a dg_prefix).  At
configs[1] (100 trajectories of a 96-token prompt, 48 new tokens) that is 1 %
of the broadcast copy's writes and a third of its footprint.  Reading the
``kv_cache`` attribute returns the reference's (L, 2, B, H, Tcap, D) tensor:
the split cache is expanded into it on first access (prefix positions filled
from the group's pages) and stays expanded.

All data movement is done by libdgattn (dg_copy4d, or the fused
dg_rope_qknorm_append in MultiHeadAttention); only the bookkeeping is Python.
"""

import torch

from diff_gpt import _native


def _grown_capacity(t1: int) -> int:
    # kv_cache.py:92-96: what is needed plus 1024, rounded up to 1024
    return ((t1 + 1024) + 1023) & ~1023


def _pages(x: torch.Tensor, t: int, t0: int = 0) -> torch.Tensor:
    """(L,2,B,H,T,D) cache (or slice) -> 4-D (L*2, B, H, t*D) view of positions
    t0 .. t0+t-1 of every page (positions and D are contiguous inside a page)."""
    L, two, B, H, _, D = x.shape
    st = x.stride()
    return x.as_strided((L * two, B, H, t * D), (st[1], st[2], st[3], 1), x.storage_offset() + t0 * st[4])


class KVCache:
    """
    Works hand-in-hand with the GPT model to maintain the KV cache.
    Note that the .pos advances automatically after the last layer of the Transformer inserts.
    """

    __slots__ = (
        "kv_shape",
        "_kv",
        "_prefix_kv",
        "pos",
        "shared_prefix",
        "pos_dev",
        "_normed",
        "_exposed",
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
        # the rows' pages: the whole (L,2,B,H,Tcap,D) cache, or, with separate
        # prefix pages, (L,2,B,H,Tcap-P,D) holding positions P.. of every row
        self._kv = torch.zeros(0)
        # (L,2,G,H,P,D) pages of a prefix shared by the rows of each group, or None
        self._prefix_kv: torch.Tensor | None = None
        self.pos = 0
        # (length, group) when rows come in groups of `group` consecutive rows
        # whose first `length` positions are identical (a batch-broadcast
        # prefill); decode attention then reads that prefix once per group --
        # from the prefix pages, or from the group's first row once expanded.
        # None otherwise.
        self.shared_prefix: tuple[int, int] | None = None
        # Device mirror of `pos` (one int32) while a captured decode step is in
        # use: the graph-replayable kernels read the position from it, and the
        # step advances both copies.  None in ordinary (eager) use.
        self.pos_dev: torch.Tensor | None = None
        # True while every key below pos was written by the model's attention
        # (RoPE + QK-norm, mha.py:44-48).  See keys_normed.
        self._normed = True
        # True once the cache tensor was handed to or taken from a caller
        self._exposed = False

    @property
    def keys_normed(self) -> bool:
        """True while every key row below pos is known to be RMS-normalised:
        each was written by the model's attention (RoPE + QK-norm,
        mha.py:44-48), and the cache tensor never passed through the
        ``kv_cache`` attribute or ``insert_kv`` (which returns views of it),
        whose holder may write keys into it in place at any later time.  The prefill kernel then runs its softmax without a
        running maximum; otherwise it keeps one."""
        return self._normed and not self._exposed

    @keys_normed.setter
    def keys_normed(self, value: bool) -> None:
        self._normed = bool(value)

    # -- the reference's tensor ------------------------------------------------
    @property
    def kv_cache(self) -> torch.Tensor:
        """The (L, 2, B, H, Tcap, D) cache tensor (kv_cache.py:25); a cache whose
        prefix lives in separate pages is expanded into it first.  The caller
        may write into it, so from here on keys_normed is False."""
        self._exposed = True
        return self._tensor()

    @kv_cache.setter
    def kv_cache(self, value: torch.Tensor) -> None:
        self._kv = value
        self._prefix_kv = None
        self._exposed = True  # contents from the caller

    def _tensor(self) -> torch.Tensor:
        """The (L, 2, B, H, Tcap, D) cache tensor for the library's own reads
        and writes (prefix pages expanded first); keys_normed is unaffected."""
        if self._prefix_kv is not None:
            self._expand()
        return self._kv

    @property
    def own_start(self) -> int:
        """First position the rows' pages hold: the prefix length when the
        prefix lives in separate pages, else 0."""
        return 0 if self._prefix_kv is None else self.shared_prefix[0]

    def nbytes(self) -> int:
        """Device bytes held (rows' pages plus prefix pages)."""
        n = self._kv.numel() * self._kv.element_size()
        if self._prefix_kv is not None:
            n += self._prefix_kv.numel() * self._prefix_kv.element_size()
        return n

    def _expand(self) -> None:
        """Turn separate prefix pages into the (L,2,B,H,Tcap,D) layout: every
        row's prefix positions filled from its group's pages, its own pages
        after them.  The prefix stays recorded as shared (read from each
        group's first row)."""
        own, pre = self._kv, self._prefix_kv
        P, group = self.shared_prefix
        L, two, B, H, cap, D = self.kv_shape
        G = pre.size(2)
        dense = torch.empty(self.kv_shape, dtype=own.dtype, device=own.device)
        ops = _native.ops()
        # prefix: (L*2*G, group, H, P*D) rows of the dense pages <- the group's page
        dst = dense.as_strided((L * two * G, group, H, P * D), (group * H * cap * D, H * cap * D, cap * D, 1))
        src = pre.reshape(L * two * G, 1, H, P * D).expand(L * two * G, group, H, P * D)
        ops.copy4d(src, dst)
        if cap > P:
            ops.copy4d(_pages(own, cap - P), _pages(dense, cap - P, P))
        self._kv, self._prefix_kv = dense, None

    def reset(self) -> None:
        if self._prefix_kv is not None:
            self._expand()  # later writes start at position 0
        self.pos = 0
        self.shared_prefix = None
        self.keys_normed = True

    def get_pos(self) -> int:
        return self.pos

    # -- prefill: batch-1 prompt cache -> num_samples rows (kv_cache.py:35-81) --
    def prefill(self, other: "KVCache") -> None:
        assert self._kv.size(0) == 0 and self._prefix_kv is None, "Cannot prefill a non-empty KV cache"
        self._fill_from(other, reuse=False)

    def _refill(self, other: "KVCache") -> None:
        """prefill() into the pages this cache already holds (same shapes,
        dtype and device as a fresh prefill would allocate), so the pointers
        a captured decode step baked in stay valid."""
        assert self._kv.size(0) != 0, "_refill needs an allocated cache"
        self._fill_from(other, reuse=True)

    def _prefill_groups(self, other: "KVCache", group: int, reuse: bool = False) -> None:
        """Prefill from a cache of G = B / group rows (one prompt per group):
        rows g*group .. g*group+group-1 start from row g of ``other``.  The
        prompts are stored once, as prefix pages; each row gets pages for its
        own positions."""
        ob = other.kv_shape[2]
        assert self.kv_shape[2] == ob * group, (
            f"Batch size mismatch: {self.kv_shape[2]} rows != {ob} prompts x {group}"
        )
        self._fill_from(other, reuse=reuse, group=group)

    def _fill_from(self, other: "KVCache", reuse: bool, group: int | None = None) -> None:
        assert other._kv.size(0) != 0, "Cannot prefill with a None KV cache"
        sl, skv, sb, sh, st, sd = self.kv_shape
        ol, okv, ob, oh, ot, od = other.kv_shape
        assert sl == ol, f"Layer count mismatch: {sl} != {ol}"
        assert skv == okv, f"K/V dimension mismatch: {skv} != {okv}"
        assert sh == oh, f"Head count mismatch: {sh} != {oh}"
        assert sd == od, f"Head dim mismatch: {sd} != {od}"
        if group is None:
            assert sb == ob or ob == 1, (
                f"Batch size mismatch: {sb} vs {ob} (other must be 1 or equal)"
            )
            group = sb if ob == 1 else 1
        assert st >= ot, f"Sequence length mismatch: {st} < {ot}"

        src = other._tensor()
        _native.require_device("KVCache.prefill", src)
        n = other.pos
        ops = _native.ops()
        split = group > 1 and n > 0
        if split:
            # the prompts once, as (L,2,G,H,n,D) prefix pages; the rows' own
            # positions n.. in pages of their own
            pre_shape = (sl, skv, ob, sh, n, sd)
            own_shape = (sl, skv, sb, sh, st - n, sd)
            if reuse:
                pre, own = self._prefix_kv, self._kv
                assert (
                    pre is not None and tuple(pre.shape) == pre_shape and tuple(own.shape) == own_shape
                    and own.dtype == src.dtype and own.device == src.device
                ), "_refill: the held pages do not match the prompt cache"
            else:
                pre = torch.empty(pre_shape, dtype=src.dtype, device=src.device)
                own = torch.empty(own_shape, dtype=src.dtype, device=src.device)
            ops.copy4d(_pages(src, n), _pages(pre, n))
            self._kv, self._prefix_kv = own, pre
            self.shared_prefix = (n, group)
        else:
            if reuse:
                dst = self._kv
                assert self._prefix_kv is None and tuple(dst.shape) == tuple(self.kv_shape) and (
                    dst.dtype == src.dtype and dst.device == src.device
                ), "_refill: the held cache does not match the prompt cache"
            else:
                self._kv = torch.empty(self.kv_shape, dtype=src.dtype, device=src.device)
                self._prefix_kv = None
            if n > 0:
                dst4 = _pages(self._kv, n)
                src4 = _pages(src, n)
                if ob == 1 and sb != 1:
                    src4 = src4.expand(dst4.shape)  # batch broadcast: 0 stride on B
                ops.copy4d(src4, dst4)
            self.shared_prefix = None
        self.pos = n
        self.keys_normed = other.keys_normed

    # -- capacity management shared by insert_kv and the fused MHA path --
    def ensure_window(
        self, T_add: int, dtype: torch.dtype, device: torch.device
    ) -> tuple[int, int]:
        """Make room for T_add more positions at ``pos``; returns (t0, t1)."""
        if self._kv.size(0) == 0:
            _native.require_device_type("KVCache", device)
            self._kv = torch.empty(self.kv_shape, dtype=dtype, device=device)
        t0, t1 = self.pos, self.pos + T_add
        if self.shared_prefix is not None and t0 < self.shared_prefix[0]:
            # rows diverge from position t0 on: only the part before it stays shared
            if self._prefix_kv is not None:
                self._expand()
            self.shared_prefix = (t0, self.shared_prefix[1]) if t0 > 0 else None
        cap = self.kv_shape[4]
        if t1 > cap:
            new_cap = _grown_capacity(t1)
            P = self.own_start
            old = self._kv
            shape = list(old.shape)
            shape[4] = new_cap - P
            grown = torch.empty(shape, dtype=old.dtype, device=old.device)
            if cap > P:
                _native.ops().copy4d(_pages(old, cap - P), _pages(grown, cap - P))
            self._kv = grown
            kv = list(self.kv_shape)
            kv[4] = new_cap
            self.kv_shape = tuple(kv)
        return t0, t1

    def layer_views(self, layer_idx: int, t1: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(B,H,t1,D) views of layer ``layer_idx``'s keys and values."""
        cache = self._tensor()
        return (
            cache[layer_idx, 0, :, :, :t1, :],
            cache[layer_idx, 1, :, :, :t1, :],
        )

    def decode_views(self, layer_idx: int):
        """What a decode step of layer ``layer_idx`` attends over: the rows'
        pages as (B, positions, H, D) views (from position own_start), and the
        shared prefix as a _native.Prefix (None without one)."""
        pages = self._kv
        k_pages = pages[layer_idx, 0].transpose(1, 2)
        v_pages = pages[layer_idx, 1].transpose(1, 2)
        if self.shared_prefix is None:
            return k_pages, v_pages, None
        P, group = self.shared_prefix
        if self._prefix_kv is None:
            return k_pages, v_pages, _native.Prefix(P, group)
        pre = self._prefix_kv
        return k_pages, v_pages, _native.Prefix(
            P, group, pre[layer_idx, 0].transpose(1, 2), pre[layer_idx, 1].transpose(1, 2), P
        )

    def advance(self, layer_idx: int, t1: int) -> None:
        """pos moves once the last layer has written its window (kv_cache.py:113-115)."""
        if layer_idx == self.kv_shape[0] - 1:
            self.pos = t1

    # -- reference entry point: copy ready-made k/v (B,H,T,D) into the cache --
    def insert_kv(
        self, layer_idx: int, k: torch.Tensor, v: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        _native.require_device("KVCache.insert_kv", k, v)
        _native.require_inference("KVCache.insert_kv", k, v)
        if self._prefix_kv is not None:
            self._expand()
        B, H, T_add, D = k.size()
        t0, t1 = self.ensure_window(T_add, k.dtype, k.device)
        cache = self._kv
        if k.dtype != cache.dtype:
            k = k.to(cache.dtype)
        if v.dtype != cache.dtype:
            v = v.to(cache.dtype)
        _native.ops().copy4d(k, cache[layer_idx, 0, :, :, t0:t1, :])
        _native.ops().copy4d(v, cache[layer_idx, 1, :, :, t0:t1, :])
        # keys from the caller, and views of the cache handed back: no norm to rely on
        self._exposed = True
        key_view, value_view = self.layer_views(layer_idx, t1)
        self.advance(layer_idx, t1)
        return key_view, value_view
