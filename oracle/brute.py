"""Textbook per-sample gradients (test infrastructure only).

One backward pass per sample gives each sample's gradient by definition; the ghost
quantities are then plain inner products of these.  Used to pin the oracle formulas and
the engine's routing (which parameter receives which dot and which train gradient).
"""
from __future__ import annotations

from typing import Callable, Dict

import torch


def per_sample_grads(model: torch.nn.Module, X: torch.Tensor, Y: torch.Tensor,
                     sample_loss: Callable, scale: float) -> Dict[str, torch.Tensor]:
    """{name: [N, *param.shape] float64} with grad_n = d(scale * sample_loss(n)) / d param.

    ``sample_loss(model, x_n, y_n)`` is the summed loss of one sample (batch of 1);
    ``scale`` is the factor the batch loss applies to it (1/N for a mean over N samples,
    1/(N*T) for a token mean).
    """
    params = [(n, p) for n, p in model.named_parameters()]
    saved = [p.requires_grad for _, p in params]
    for _, p in params:
        p.requires_grad_(True)
    out: Dict[str, list] = {n: [] for n, _ in params}
    try:
        for i in range(X.shape[0]):
            model.zero_grad(set_to_none=True)
            loss = sample_loss(model, X[i:i + 1], Y[i:i + 1]) * scale
            loss.backward()
            for n, p in params:
                g = p.grad
                out[n].append(torch.zeros_like(p, dtype=torch.float64) if g is None
                              else g.detach().double().clone())
    finally:
        for (_, p), r in zip(params, saved):
            p.requires_grad_(r)
        model.zero_grad(set_to_none=True)
    return {n: torch.stack(v) for n, v in out.items()}


def pairwise_dots(grads: torch.Tensor, n_val: int) -> torch.Tensor:
    """[n_train] <g_i, sum_j g_j> over the last n_val rows as val (reference layout)."""
    N = grads.shape[0]
    flat = grads.reshape(N, -1)
    tr, va = flat[:N - n_val], flat[N - n_val:]
    return tr @ va.sum(0)


def pair_matrix(grads: torch.Tensor, n_val: int) -> torch.Tensor:
    """[n_val, n_train] <g_i, g_j>."""
    N = grads.shape[0]
    flat = grads.reshape(N, -1)
    tr, va = flat[:N - n_val], flat[N - n_val:]
    return va @ tr.T


def train_mean(grads: torch.Tensor, n_val: int, N_scale: float) -> torch.Tensor:
    """The reference's train gradient from per-sample grads of the N-mean loss:
    sum over train rows of (N * g_i) / n_train."""
    n_t = grads.shape[0] - n_val
    return grads[:n_t].sum(0) * N_scale / n_t
