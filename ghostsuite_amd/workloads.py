"""Workload models for the benchmark configurations (random init, synthetic data).

These are the callers of the hot path, not part of it: an MLP, a GPT-2 with
nn.Linear projections, tied lm_head and per-sample position ids (configs[2] GPT-2-small,
configs[3] GPT-2-medium shape), and a rotary GPT-NeoX-style model (configs[4] Pythia-1B
shape).  Embeddings listed in ``ghost_embeddings`` receive the dummy bias of the engine's
forward swapper, which keeps the autograd graph alive when every weight is frozen.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn


class MLP(nn.Module):
    """Linear 512 -> 1024 -> ReLU -> 1024 -> ReLU -> 10."""

    def __init__(self, dims=(512, 1024, 1024, 10)):
        super().__init__()
        layers = []
        for i in range(len(dims) - 1):
            layers.append(nn.Linear(dims[i], dims[i + 1]))
            if i < len(dims) - 2:
                layers.append(nn.ReLU())
        self.net = nn.Sequential(*layers)

    def forward(self, x):
        return self.net(x)


@dataclass
class LMConfig:
    n_layer: int = 12
    n_head: int = 12
    d_model: int = 768
    d_mlp: int = 3072
    vocab: int = 50257
    n_ctx: int = 1024
    rotary: bool = False
    tied: bool = True
    rotary_pct: float = 0.25


GPT2_SMALL = LMConfig()
GPT2_MEDIUM = LMConfig(n_layer=24, n_head=16, d_model=1024, d_mlp=4096)
PYTHIA_1B = LMConfig(n_layer=16, n_head=8, d_model=2048, d_mlp=8192, vocab=50304, n_ctx=2048,
                     rotary=True, tied=False)


def _attention(q, k, v):
    """Causal attention through the fused flash / memory-efficient SDPA kernels only."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    if q.is_cuda:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, is_causal=True)
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                          is_causal=True).to(q.dtype)


def _rotary(x, cos, sin, n_rot):
    xr, xp = x[..., :n_rot], x[..., n_rot:]
    x1, x2 = xr[..., : n_rot // 2], xr[..., n_rot // 2:]
    rot = torch.cat((-x2, x1), dim=-1)
    return torch.cat((xr * cos + rot * sin, xp), dim=-1)


class Block(nn.Module):
    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.cfg = cfg
        d = cfg.d_model
        self.ln_1 = nn.LayerNorm(d)
        self.qkv = nn.Linear(d, 3 * d)
        self.proj = nn.Linear(d, d)
        self.ln_2 = nn.LayerNorm(d)
        self.fc = nn.Linear(d, cfg.d_mlp)
        self.fc_out = nn.Linear(cfg.d_mlp, d)

    def forward(self, x, rope=None):
        B, T, d = x.shape
        H = self.cfg.n_head
        q, k, v = self.qkv(self.ln_1(x)).split(d, dim=-1)
        q = q.view(B, T, H, d // H).transpose(1, 2)
        k = k.view(B, T, H, d // H).transpose(1, 2)
        v = v.view(B, T, H, d // H).transpose(1, 2)
        if rope is not None:
            cos, sin, n_rot = rope
            q = _rotary(q, cos, sin, n_rot)
            k = _rotary(k, cos, sin, n_rot)
        y = _attention(q.contiguous(), k.contiguous(), v.contiguous())
        x = x + self.proj(y.transpose(1, 2).reshape(B, T, d))
        return x + self.fc_out(F.gelu(self.fc(self.ln_2(x)), approximate="tanh"))


class CausalLM(nn.Module):
    """GPT-2 (learned positions, tied lm_head) or rotary GPT-NeoX-style (untied embed_out)."""

    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.cfg = cfg
        self.wte = nn.Embedding(cfg.vocab, cfg.d_model)
        if not cfg.rotary:
            self.wpe = nn.Embedding(cfg.n_ctx, cfg.d_model)
        self.h = nn.ModuleList([Block(cfg) for _ in range(cfg.n_layer)])
        self.ln_f = nn.LayerNorm(cfg.d_model)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab, bias=False)
        if cfg.tied:
            self.lm_head.weight = self.wte.weight
        self.ghost_embeddings = ("wte",) if cfg.rotary else ("wte", "wpe")
        self.apply(self._init)

    @staticmethod
    def _init(m):
        if isinstance(m, (nn.Linear, nn.Embedding)):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
        if isinstance(m, nn.Linear) and m.bias is not None:
            nn.init.zeros_(m.bias)

    def _rope(self, T, device, dtype):
        hd = self.cfg.d_model // self.cfg.n_head
        n_rot = int(hd * self.cfg.rotary_pct)
        inv = 1.0 / (10000 ** (torch.arange(0, n_rot, 2, device=device).float() / n_rot))
        t = torch.arange(T, device=device).float()
        fr = torch.outer(t, inv)
        emb = torch.cat((fr, fr), dim=-1)
        return emb.cos().to(dtype), emb.sin().to(dtype), n_rot

    def forward(self, input_ids, labels=None):
        B, T = input_ids.shape
        x = self.wte(input_ids)
        rope = None
        if self.cfg.rotary:
            rope = self._rope(T, input_ids.device, x.dtype)
        else:
            # per-sample position ids so the position embedding's hook sees [B, T]
            pos = torch.arange(T, device=input_ids.device).unsqueeze(0).repeat(B, 1)
            x = x + self.wpe(pos)
        for blk in self.h:
            x = blk(x, rope)
        logits = self.lm_head(self.ln_f(x))
        if labels is None:
            return logits
        return F.cross_entropy(logits.float().view(-1, logits.shape[-1]), labels.reshape(-1))


def synthetic_tokens(n_rows: int, T: int, vocab: int, seed: int, device="cpu"):
    """Uniform token ids and next-token labels (ids shifted by one, last label random)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (n_rows, T + 1), generator=g)
    return ids[:, :T].contiguous().to(device), ids[:, 1:].contiguous().to(device)


def lm_flops_per_step(cfg: LMConfig, n_rows: int, T: int) -> float:
    """6 * params * tokens + attention (fwd+bwd), the plain-backprop work of one step."""
    d, L = cfg.d_model, cfg.n_layer
    params = L * (4 * d * d + 2 * d * cfg.d_mlp) + cfg.vocab * d
    attn = L * 2 * 2 * T * T * d * 3  # QK^T and PV, fwd + 2x bwd
    return 6.0 * params * n_rows * T + attn * n_rows
