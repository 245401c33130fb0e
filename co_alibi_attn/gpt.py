"""GPT training step with Co-ALiBi attention: the caller of the attention hot path.

The reference has no model code; its benchmark configs name this one (12 layers,
d_model 768, 12 heads of 64, no positional embeddings, vocab 50304, B=8, S=1024,
bf16 autocast, AdamW, one fwd+bwd+step).  Positions enter only through the
Co-ALiBi penalty of ``co_alibi_attention`` (the 12-head slope table uses the
non-power-of-two branch of ``_get_coalibi_slopes``).

The block is a standard pre-norm transformer block: LayerNorm, fused QKV
projection, causal Co-ALiBi attention, output projection, residual; LayerNorm,
GELU MLP (4x), residual.  The LM head is tied to the token embedding.

``attention`` is injectable so tests can run the same model on the CPU with a
reference attention; the default is the native ``co_alibi_attention``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable

import torch
import torch.nn as nn
import torch.nn.functional as F

from .co_alibi_attn import co_alibi_attention


@dataclass(frozen=True)
class GPTConfig:
    n_layer: int = 12
    n_head: int = 12
    d_model: int = 768
    vocab: int = 50304
    mlp_ratio: int = 4
    bias_max: float = 8.0


AttentionFn = Callable[..., torch.Tensor]


class CausalCoALiBiAttention(nn.Module):
    def __init__(self, cfg: GPTConfig, attention: AttentionFn):
        super().__init__()
        self.n_head = cfg.n_head
        self.head_dim = cfg.d_model // cfg.n_head
        self.bias_max = cfg.bias_max
        self.qkv = nn.Linear(cfg.d_model, 3 * cfg.d_model, bias=False)
        self.proj = nn.Linear(cfg.d_model, cfg.d_model, bias=False)
        self.attention = attention

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, S, C = x.shape
        qkv = self.qkv(x).view(B, S, 3, self.n_head, self.head_dim)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))  # (B, H, S, D) views
        y = self.attention(q, k, v, causal=True, bias_max=self.bias_max)
        return self.proj(y.transpose(1, 2).reshape(B, S, C))


class Block(nn.Module):
    def __init__(self, cfg: GPTConfig, attention: AttentionFn):
        super().__init__()
        self.ln1 = nn.LayerNorm(cfg.d_model)
        self.attn = CausalCoALiBiAttention(cfg, attention)
        self.ln2 = nn.LayerNorm(cfg.d_model)
        self.fc = nn.Linear(cfg.d_model, cfg.mlp_ratio * cfg.d_model)
        self.out = nn.Linear(cfg.mlp_ratio * cfg.d_model, cfg.d_model)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln1(x))
        return x + self.out(F.gelu(self.fc(self.ln2(x)), approximate="tanh"))


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig = GPTConfig(), attention: AttentionFn = co_alibi_attention):
        super().__init__()
        self.cfg = cfg
        self.wte = nn.Embedding(cfg.vocab, cfg.d_model)
        self.blocks = nn.ModuleList(Block(cfg, attention) for _ in range(cfg.n_layer))
        self.ln_f = nn.LayerNorm(cfg.d_model)
        self.apply(self._init)
        # GPT-2 style scaled init of the residual projections.
        for name, p in self.named_parameters():
            if name.endswith("attn.proj.weight") or name.endswith("out.weight"):
                nn.init.normal_(p, mean=0.0, std=0.02 / math.sqrt(2 * cfg.n_layer))

    @staticmethod
    def _init(m: nn.Module) -> None:
        if isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
            if m.bias is not None:
                nn.init.zeros_(m.bias)
        elif isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)

    def forward(self, idx: torch.Tensor, targets: torch.Tensor | None = None):
        x = self.wte(idx)
        for blk in self.blocks:
            x = blk(x)
        logits = F.linear(self.ln_f(x), self.wte.weight)  # tied LM head
        if targets is None:
            return logits
        loss = F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.view(-1))
        return logits, loss

    def n_params(self) -> int:
        return sum(p.numel() for p in self.parameters())


def make_optimizer(model: GPT, lr: float = 6e-4, weight_decay: float = 0.1) -> torch.optim.Optimizer:
    """AdamW with weight decay on matrices only (embeddings and linear weights)."""
    decay = [p for p in model.parameters() if p.dim() >= 2]
    no_decay = [p for p in model.parameters() if p.dim() < 2]
    groups = [{"params": decay, "weight_decay": weight_decay}, {"params": no_decay, "weight_decay": 0.0}]
    return torch.optim.AdamW(groups, lr=lr, betas=(0.9, 0.95), eps=1e-8)


def synthetic_batch(cfg: GPTConfig, batch: int, seq: int, seed: int = 0, device="cpu"):
    """Uniform-random token ids (inputs and next-token targets), drawn on the CPU."""
    gen = torch.Generator().manual_seed(seed)
    tok = torch.randint(0, cfg.vocab, (batch, seq + 1), generator=gen)
    return tok[:, :-1].contiguous().to(device), tok[:, 1:].contiguous().to(device)


def train_step(model: GPT, opt: torch.optim.Optimizer, idx: torch.Tensor, targets: torch.Tensor,
               autocast_dtype: torch.dtype | None = torch.bfloat16) -> torch.Tensor:
    """One forward + backward + AdamW step; returns the (detached) loss."""
    opt.zero_grad(set_to_none=True)
    if autocast_dtype is None:
        _, loss = model(idx, targets)
    else:
        with torch.autocast(device_type=idx.device.type, dtype=autocast_dtype):
            _, loss = model(idx, targets)
    loss.backward()
    opt.step()
    return loss.detach()
