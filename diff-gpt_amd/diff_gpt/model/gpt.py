"""GPT over the MI355X attention path (src/diff_gpt/model/gpt.py:15-242).

Same constructor, parameter names (state_dicts load both ways), parameter
creation order (so a seeded construction gives the same weights), forward
signature and generation API as the reference.  Inference only: the HIP
kernels have no backward, so a forward that would need autograd raises.
"""

from abc import ABC, abstractmethod

import torch
import torch.nn as nn
from torch.nn import functional as F

from diff_gpt import _native
from diff_gpt.model.block import Block
from diff_gpt.model.kv_cache import KVCache
from diff_gpt.model.rms_norm import rms_norm
from diff_gpt.model.rope import precompute_freqs_cis
from diff_gpt.sampler.sampler import Sampler
from diff_gpt.sampler.temperature import TemperatureSampler, draw_one


def _ordinal_target_table(V: int, sigma: float, dtype: torch.dtype, device) -> torch.Tensor:
    """(V, V) table whose row t is the soft target for token t: a discretised
    Gaussian over the bin indices centred on t with standard deviation sigma
    (in bins), normalised to sum to 1."""
    bins = torch.arange(V, device=device, dtype=torch.float64)
    z = (bins[None, :] - bins[:, None]) / sigma
    return torch.softmax(-0.5 * z * z, dim=-1).to(dtype)


def _ordinal_soft_ce(
    logits: torch.Tensor,
    targets: torch.Tensor,
    sigma: float,
    ignore_index: int = -100,
) -> torch.Tensor:
    """Mean over the rows whose target is not ignore_index of the cross-entropy
    between the row's log-softmax and its Gaussian soft target (the training
    loss of gpt.py:15-35 for label_smoothing_sigma > 0); 0 when every row is
    ignored."""
    valid = targets != ignore_index
    soft = _ordinal_target_table(logits.size(-1), sigma, logits.dtype, logits.device)
    rows = soft[torch.where(valid, targets, 0)]
    per_row = -(rows * F.log_softmax(logits, dim=-1)).sum(dim=-1)
    return torch.where(valid, per_row, 0.0).sum() / valid.sum().clamp(min=1)


class BaseGPT(nn.Module, ABC):
    def __init__(
        self,
        block_size: int,
        vocab_size: int,
        n_embd: int,
        n_head: int,
        n_layer: int,
    ) -> None:
        super().__init__()
        self.block_size = block_size
        self.vocab_size = vocab_size
        self.n_embd = n_embd
        self.n_head = n_head
        self.n_layer = n_layer

    @abstractmethod
    def forward(
        self,
        idx: torch.Tensor,
        targets: torch.Tensor | None = None,
        kv_cache: KVCache | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        pass

    @abstractmethod
    def generate(
        self,
        idx: torch.Tensor,
        max_new_tokens: int,
        sampler: Sampler | None,
        seed: int | None = None,
    ) -> torch.Tensor:
        pass

    @property
    @abstractmethod
    def device_type(self) -> str:
        pass


class GPT(BaseGPT):
    def __init__(
        self,
        vocab_size: int,
        n_embd: int = 64,
        block_size: int = 32,
        n_head: int = 4,
        n_layer: int = 4,
        rope_theta: float = 10000,
        swiglu_alpha: float = 1.702,
        swiglu_limit: float = 7.0,
        use_checkpoint: bool = True,
        logit_softcap: float = 15.0,
        pad_vocab_size_to: int = 64,
        attn_res_layers_per_block: int = 1,
        label_smoothing_sigma: float = 0.0,
    ) -> None:
        super().__init__(
            block_size=block_size,
            vocab_size=vocab_size,
            n_embd=n_embd,
            n_head=n_head,
            n_layer=n_layer,
        )
        assert logit_softcap >= 0, "logit_softcap must be non-negative (0 disables it)"
        assert label_smoothing_sigma >= 0, (
            "label_smoothing_sigma must be non-negative (0 disables it)"
        )
        assert pad_vocab_size_to >= 1, "pad_vocab_size_to must be >= 1"
        assert attn_res_layers_per_block >= 1, "attn_res_layers_per_block must be >= 1"
        assert vocab_size % pad_vocab_size_to == 0, (
            f"vocab_size ({vocab_size}) must be a multiple of "
            f"pad_vocab_size_to ({pad_vocab_size_to}); pad it in the encoder"
        )
        self.token_embedding_table = nn.Embedding(vocab_size, n_embd)
        self.blocks = nn.ModuleList(
            Block(
                n_embd=n_embd,
                n_head=n_head,
                swiglu_alpha=swiglu_alpha,
                swiglu_limit=swiglu_limit,
                layer_idx=i,
                layers_per_block=attn_res_layers_per_block,
            )
            for i in range(n_layer)
        )
        # lm_head is created (consuming the seeded RNG) and then tied
        self.lm_head = nn.Linear(n_embd, vocab_size, bias=False)
        self.lm_head.weight = self.token_embedding_table.weight
        # RoPE table for 2*block_size positions; not saved in the state_dict
        self.register_buffer(
            "freqs_cis",
            precompute_freqs_cis(n_embd // n_head, block_size * 2, theta=rope_theta),
            persistent=False,
        )
        self.use_checkpoint = use_checkpoint
        self.logit_softcap = logit_softcap
        self.label_smoothing_sigma = label_smoothing_sigma

    def _head(self, partial: torch.Tensor, argmax_out: torch.Tensor | None,
              xn: torch.Tensor | None = None) -> torch.Tensor:
        """rms_norm -> tied lm_head -> softcap (gpt.py:180-186): one dg_lm_head
        launch after the norm (xn, when the last layer's launch wrote it),
        which also writes each row's argmax into argmax_out (B, T) when given;
        F.linear + dg_softcap (+ torch.argmax) for shapes it does not take."""
        if xn is None:
            xn = rms_norm(partial)
        B, T, C = xn.shape
        V = self.lm_head.weight.size(0)
        cap = float(self.logit_softcap)
        logits = torch.empty((B, T, V), dtype=xn.dtype, device=xn.device)
        ids = None if argmax_out is None else argmax_out.view(B * T)
        if _native.lm_head_(xn.view(B * T, C), self.lm_head.weight, cap, logits.view(B * T, V), ids):
            return logits
        logits = self.lm_head(xn)
        if cap > 0:
            _native.ops().softcap_(logits, cap)  # cap * tanh(logits / cap)
        if argmax_out is not None:
            argmax_out.copy_(torch.argmax(logits, dim=-1))
        return logits

    def _embed(self, idx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor | None]:
        """x = rms_norm(token_embedding_table(idx)) (gpt.py:154-155) and, when there
        is a layer 0, rms_norm(x): one dg_embed_norm launch.  An id outside the
        vocabulary gives a NaN row (nn.Embedding raises).  fp64 tables take
        nn.Embedding and the RMSNorm kernel."""
        table = self.token_embedding_table.weight
        _native.require_device("GPT", idx, table)
        _native.require_inference("GPT", table)
        C = table.size(1)
        x = torch.empty((*idx.shape, C), dtype=table.dtype, device=table.device)
        xn0 = torch.empty_like(x) if self.blocks else None
        if _native.embed_norm_(idx, table, x, xn0):
            return x, xn0
        return rms_norm(self.token_embedding_table(idx)), None

    def forward(
        self,
        idx: torch.Tensor,
        targets: torch.Tensor | None = None,
        kv_cache: KVCache | None = None,
        *,
        _argmax_out: torch.Tensor | None = None,
        _last_only: bool = False,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """gpt.py:140-200.  _argmax_out (B, T) int64, when given, receives the
        first maximum of every logits row (greedy sampling without a separate
        argmax launch).  _last_only returns the (B, 1, V) logits of the last
        position only (a prefill whose caller reads no others; _argmax_out is
        then (B, 1)): every layer still attends and caches every position, but
        the last layer's work after its attention and the head run for that
        position alone."""
        B, T = idx.shape
        assert not (_last_only and targets is not None), "_last_only returns the last position's logits alone"
        start = 0 if kv_cache is None else kv_cache.get_pos()
        end = start + T
        assert end <= self.freqs_cis.shape[0]
        if kv_cache is not None and kv_cache.pos_dev is not None:
            # captured decode step: the kernels index the whole table with the
            # position they read on the device
            freqs_cis = self.freqs_cis
        else:
            freqs_cis = self.freqs_cis[start:end].view(1, T, 1, -1, 2)

        # the normalised embedding and, when layer 0 reads it, layer 0's
        # attention input rms_norm(x) (its one-block mixture) in one launch
        x, xn0 = self._embed(idx)
        # Block-AttnRes state: the normalised embedding is block 0 and also the
        # first partial sum
        blocks: tuple[torch.Tensor, ...] = (x,)
        partial = x
        last = len(self.blocks) - 1
        # the head's input rms_norm(partial), written by the last layer
        xn_head = None
        if self.blocks:
            xn_head = torch.empty((B, 1 if _last_only else T, x.size(-1)), dtype=x.dtype, device=x.device)
        for i, block in enumerate(self.blocks):
            blocks, partial = block(blocks, partial, freqs_cis=freqs_cis, kv_cache=kv_cache,
                                    _last_only=_last_only and i == last, _xn=xn0 if i == 0 else None,
                                    _xn_out=xn_head if i == last else None)
        if _last_only and not self.blocks:
            partial = partial[:, -1:]

        logits = self._head(partial, _argmax_out, xn_head)

        loss = None
        if targets is not None:
            flat_logits = logits.view(B * T, -1)
            flat_targets = targets.view(B * T)
            if self.label_smoothing_sigma > 0:
                loss = _ordinal_soft_ce(
                    flat_logits, flat_targets, sigma=self.label_smoothing_sigma
                )
            else:
                loss = F.cross_entropy(flat_logits, flat_targets)
        return logits, loss

    @torch.inference_mode()
    def generate(
        self,
        idx: torch.Tensor,
        max_new_tokens: int,
        sampler: Sampler | None,
        seed: int | None = None,
    ) -> torch.Tensor:
        """Cache-free sliding-window sampling (gpt.py:202-237): every step
        re-runs the last block_size tokens through the causal prefill path."""
        device = idx.device
        rng = None
        if seed is not None:
            rng = torch.Generator(device=device)
            rng.manual_seed(seed)
        B, T = idx.shape
        out = torch.zeros((B, T + max_new_tokens), dtype=torch.int64, device=device)
        out[:, :T] = idx
        # greedy: the argmax comes out of the lm_head launch (temperature.py:22-23)
        greedy = type(sampler) is TemperatureSampler and sampler.temperature == 0
        for cur in range(T, T + max_new_tokens):
            window = out[:, max(0, cur - self.block_size) : cur]
            # only the last position's logits are read
            if greedy:
                am = torch.empty((B, 1), dtype=torch.int64, device=device)
                self(window, _argmax_out=am, _last_only=True)
                out[:, cur] = am[:, -1]
                continue
            logits, _ = self(window, _last_only=True)
            last = logits[:, -1]
            if sampler is not None:
                nxt = sampler(last, rng=rng)
            else:
                nxt = draw_one(F.softmax(last, dim=-1), rng)
            out[:, cur] = nxt.squeeze()
        return out

    @property
    def device_type(self) -> str:
        return str(self.freqs_cis.device.type)
