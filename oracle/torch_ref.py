"""torch-on-CPU restatement of the reference model path (test infrastructure only).

A functional forward over a GPT state_dict with the reference's own library
calls: F.scaled_dot_product_attention with its three mask branches
(mha.py:61-81), F.rms_norm (rms_norm.py:7), the float32 interleaved-pair
rotation (rope.py:20-27), Block-AttnRes (block.py:10-107), clamped SwiGLU
(swi_glu.py:11-19), tied lm_head and tanh softcap (gpt.py:140-186), and a KV
cache with the reference's append / pos rules (kv_cache.py:83-116).

Pinned by: its own self-consistency checks in tests/test_oracle.py -- the
KV-cache step-by-step logits equal the full causal forward (the invariant of
test_gpt.py:34-76 and test_mha.py:80-119), the chunked branch equals the full
forward (test_mha.py:122-158), and its attention equals
oracle.numerics.attention_f64.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class ModelConfig:
    vocab_size: int
    n_embd: int
    block_size: int
    n_head: int
    n_layer: int
    rope_theta: float = 10000.0
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 7.0
    logit_softcap: float = 15.0
    attn_res_layers_per_block: int = 1

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head


def freqs_table(dim: int, end: int, theta: float) -> torch.Tensor:
    """rope.py:30-44 with the same torch ops (fp32 on the CPU)."""
    w = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32)[: dim // 2] / dim))
    ang = torch.outer(torch.arange(end, dtype=torch.float32), w)
    return torch.stack([ang.cos(), ang.sin()], dim=-1)


def rope(x: torch.Tensor, fc: torch.Tensor) -> torch.Tensor:
    """rope.py:20-27."""
    xp = x.float().reshape(*x.shape[:-1], -1, 2)
    re, im = xp[..., 0], xp[..., 1]
    c, s = fc[..., 0], fc[..., 1]
    out = torch.stack([re * c - im * s, re * s + im * c], dim=-1).flatten(-2)
    return out.type_as(x)


def rms(x: torch.Tensor) -> torch.Tensor:
    return F.rms_norm(x, (x.size(-1),))


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """mha.py:61-81 on (B,H,T,D) tensors."""
    Tq, Tk = q.size(2), k.size(2)
    if Tq == Tk:
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)
    if Tq == 1:
        return F.scaled_dot_product_attention(q, k, v, is_causal=False)
    mask = torch.ones((Tq, Tk), dtype=torch.bool).tril(diagonal=Tk - Tq)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)


class RefCache:
    """(L, 2, B, H, Tcap, D) cache with the reference's insert / pos rules."""

    def __init__(self, B: int, H: int, T: int, D: int, L: int):
        self.shape = (L, 2, B, H, T, D)
        self.data: torch.Tensor | None = None
        self.pos = 0

    def insert(self, layer: int, k: torch.Tensor, v: torch.Tensor):
        if self.data is None:
            self.data = torch.empty(self.shape, dtype=k.dtype)
        t0, t1 = self.pos, self.pos + k.size(2)
        if t1 > self.data.size(4):
            cap = ((t1 + 1024) + 1023) & ~1023
            extra = list(self.data.shape)
            extra[4] = cap - self.data.size(4)
            self.data = torch.cat([self.data, torch.empty(extra, dtype=k.dtype)], dim=4)
        self.data[layer, 0, :, :, t0:t1] = k
        self.data[layer, 1, :, :, t0:t1] = v
        if layer == self.data.size(0) - 1:
            self.pos = t1
        return self.data[layer, 0, :, :, :t1], self.data[layer, 1, :, :, :t1]

    def broadcast_from(self, other: "RefCache"):
        self.data = torch.empty(self.shape, dtype=other.data.dtype)
        n = other.pos
        self.data[..., :n, :] = other.data[..., :n, :]
        self.pos = n


def attention_layer(p: dict, pre: str, cfg: ModelConfig, layer: int, x: torch.Tensor,
                    fc: torch.Tensor, cache: RefCache | None) -> torch.Tensor:
    """mha.py:31-86."""
    B, T, C = x.shape
    H, D = cfg.n_head, cfg.head_dim
    q = (x @ p[pre + "c_q.weight"].T).view(B, T, H, D)
    k = (x @ p[pre + "c_k.weight"].T).view(B, T, H, D)
    v = (x @ p[pre + "c_v.weight"].T).view(B, T, H, D)
    g = x @ p[pre + "c_g.weight"].T
    q, k = rms(rope(q, fc)), rms(rope(k, fc))
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if cache is not None:
        k, v = cache.insert(layer, k, v)
    y = sdpa(q, k, v)
    y = y.transpose(1, 2).contiguous().view(B, T, C) * torch.sigmoid(g)
    return y @ p[pre + "c_proj.weight"].T


def attn_res(blocks, partial, w: torch.Tensor) -> torch.Tensor:
    """block.py:10-44."""
    if len(blocks) == 1 and partial is blocks[0]:
        return partial
    V = torch.stack([*blocks, partial], dim=0)
    wts = rms(V).matmul(w.view(-1)).softmax(dim=0).unsqueeze(-1)
    return (wts * V).sum(dim=0)


def mlp(p: dict, pre: str, cfg: ModelConfig, x: torch.Tensor) -> torch.Tensor:
    """feed_forward.py:7-18 + swi_glu.py:11-19."""
    h = x @ p[pre + "net.0.weight"].T
    gl = h[..., ::2].clamp(max=cfg.swiglu_limit)
    ln = h[..., 1::2].clamp(min=-cfg.swiglu_limit, max=cfg.swiglu_limit)
    h = gl * torch.sigmoid(cfg.swiglu_alpha * gl) * (ln + 1)
    return h @ p[pre + "net.2.weight"].T


def forward(p: dict, cfg: ModelConfig, idx: torch.Tensor, cache: RefCache | None = None,
            fc_table: torch.Tensor | None = None) -> torch.Tensor:
    """GPT.forward (gpt.py:140-186) -> logits (B, T, V)."""
    B, T = idx.shape
    start = 0 if cache is None else cache.pos
    if fc_table is None:
        fc_table = freqs_table(cfg.head_dim, 2 * cfg.block_size, cfg.rope_theta)
    dt = p["token_embedding_table.weight"].dtype
    fc = fc_table.to(dt)[start:start + T].view(1, T, 1, -1, 2)
    x = rms(p["token_embedding_table.weight"][idx])
    blocks, partial = (x,), x
    for i in range(cfg.n_layer):
        pre = f"blocks.{i}."
        h = attn_res(blocks, partial, p[pre + "attn_res_proj.weight"])
        boundary = (i + 1) % cfg.attn_res_layers_per_block == 0
        if boundary:
            blocks = (*blocks, partial)
        a = attention_layer(p, pre + "sa.", cfg, i, rms(h), fc, cache)
        partial = a if boundary else partial + a
        h = attn_res(blocks, partial, p[pre + "mlp_res_proj.weight"])
        partial = partial + mlp(p, pre + "ffwd.", cfg, rms(h))
    logits = rms(partial) @ p["token_embedding_table.weight"].T
    if cfg.logit_softcap > 0:
        logits = cfg.logit_softcap * torch.tanh(logits / cfg.logit_softcap)
    return logits


@torch.no_grad()
def greedy_decode(p: dict, cfg: ModelConfig, prompts: torch.Tensor, steps: int,
                  forced: list[list[int]] | None = None):
    """Batched KV-cache greedy decode driven like test_gpt.py:34-76: one prefill
    of (B, T) prompts, then ``steps`` single-token forwards, feeding back the
    argmax (or ``forced[s]`` per row when given).  Returns (tokens (B, steps),
    logits list [(B, V)] of the distribution each token was taken from)."""
    B, T = prompts.shape
    cache = RefCache(B, cfg.n_head, T + steps, cfg.head_dim, cfg.n_layer)
    table = freqs_table(cfg.head_dim, 2 * cfg.block_size, cfg.rope_theta)
    logits = forward(p, cfg, prompts, cache, table)[:, -1]
    toks, outs = [], []
    for s in range(steps):
        outs.append(logits)
        nxt = logits.argmax(dim=-1) if forced is None else torch.tensor(forced[s])
        toks.append(nxt)
        logits = forward(p, cfg, nxt[:, None], cache, table)[:, -1]
    return torch.stack(toks, dim=1), outs
