"""A small GPT for model-level tests (test infrastructure, not part of the package).

Module structure -- and therefore ``parameters()`` order, which fixes DDP's
bucket layout and FSDP's unit layout -- follows the reference model
(minidist/models/gpt.py:153-224): ``Embedding`` holds a ``wte`` embedding
module and its own ``wpe`` parameter, blocks are pre-norm (ln1, attn.qkv,
attn.proj, ln2, mlp.fc, mlp.proj), and ``LMHead`` is ln_f plus an untied,
bias-free projection.  Attention math runs in float32.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn


@dataclass
class Config:
    vocab_size: int = 64
    block_size: int = 16
    n_layer: int = 2
    n_head: int = 4
    n_embd: int = 32


class Attention(nn.Module):
    def __init__(self, c: Config):
        super().__init__()
        self.n_head, self.hd = c.n_head, c.n_embd // c.n_head
        self.qkv = nn.Linear(c.n_embd, 3 * c.n_embd)
        self.proj = nn.Linear(c.n_embd, c.n_embd)

    def forward(self, x):
        B, S, _ = x.shape
        q, k, v = self.qkv(x).view(B, S, self.n_head, 3, self.hd).unbind(dim=3)
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))
        att = (q.float() @ k.float().transpose(-1, -2).contiguous()) / self.hd**0.5
        mask = torch.ones(S, S, dtype=torch.bool, device=x.device).tril()
        att = att.masked_fill(~mask, float("-inf")).softmax(dim=-1)
        y = (att @ v.float()).to(x.dtype).transpose(1, 2).reshape(B, S, -1)
        return self.proj(y)


class MLP(nn.Module):
    def __init__(self, c: Config):
        super().__init__()
        self.fc = nn.Linear(c.n_embd, 4 * c.n_embd)
        self.proj = nn.Linear(4 * c.n_embd, c.n_embd)

    def forward(self, x):
        return self.proj(F.gelu(self.fc(x), approximate="tanh"))


class Block(nn.Module):
    def __init__(self, c: Config):
        super().__init__()
        self.ln1 = nn.LayerNorm(c.n_embd)
        self.attn = Attention(c)
        self.ln2 = nn.LayerNorm(c.n_embd)
        self.mlp = MLP(c)

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.mlp(self.ln2(x))


class Embedding(nn.Module):
    def __init__(self, c: Config):
        super().__init__()
        self.wte = nn.Embedding(c.vocab_size, c.n_embd)
        self.wpe = nn.Parameter(torch.randn(c.block_size, c.n_embd) * 0.02)

    def forward(self, ids):
        return self.wte(ids) + self.wpe[: ids.size(1)]


class LMHead(nn.Module):
    def __init__(self, c: Config):
        super().__init__()
        self.ln_f = nn.LayerNorm(c.n_embd)
        self.head = nn.Linear(c.n_embd, c.vocab_size, bias=False)

    def forward(self, x):
        return self.head(self.ln_f(x))


class GPT(nn.Module):
    def __init__(self, c: Config, seed: int = 0):
        super().__init__()
        torch.manual_seed(seed)
        self.config = c
        self.embedding = Embedding(c)
        self.blocks = nn.ModuleList([Block(c) for _ in range(c.n_layer)])
        self.lm_head = LMHead(c)

    def forward(self, ids, targets=None):
        x = self.embedding(ids)
        for b in self.blocks:
            x = b(x)
        logits = self.lm_head(x)
        if targets is None:
            return logits
        return logits, F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.view(-1))


def batch(c: Config, n: int, seed: int = 42):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, c.vocab_size, (n, c.block_size), generator=g)
    tgt = torch.randint(0, c.vocab_size, (n, c.block_size), generator=g)
    return ids, tgt
