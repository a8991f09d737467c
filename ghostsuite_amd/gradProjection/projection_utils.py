"""Projection set-up on the host: (k_i, k_o) choice and projection matrices.

Mirrors ghostEngines/gradProjection/projection_utils.py: the same integer rule for
(k_i, k_o), the same generator seeding per matrix and the same N(0, 1/rows) /
Rademacher / row-orthonormal constructions.  Matrices are drawn from a CPU generator
and moved to the model's device, so a given seed yields the same P on every machine (the
reference draws on the model's device; its CUDA stream of random numbers cannot be
reproduced on ROCm).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn


def choose_ki_ko(n_i: int, n_o: int, k_total: int, k_min: int = 1) -> Tuple[int, int]:
    """k_i/k_o ~ sqrt(n_o/n_i), k_i*k_o ~ k_total, both >= k_min; then a +-2 local search that
    only accepts strict improvements (reference projection_utils.py:12-66)."""
    if min(n_i, n_o) <= 0 or k_total <= 0:
        raise ValueError(f"Invalid dimensions for projection: n_i={n_i}, n_o={n_o}, "
                         f"k_total={k_total}")
    if k_min > min(n_i, n_o):
        raise ValueError(f"k_min={k_min} exceeds layer dimensions (n_i={n_i}, n_o={n_o})")
    ratio = math.sqrt(n_o / max(1, n_i))
    k_i = max(k_min, min(n_i, max(1, int(round(math.sqrt(k_total) * ratio)))))
    k_o = max(k_min, min(n_o, max(1, k_total // k_i)))
    best, best_err = (k_i, k_o), abs(k_i * k_o - k_total)
    for di in (-2, -1, 0, 1, 2):
        for dj in (-2, -1, 0, 1, 2):
            ki, ko = k_i + di, k_o + dj
            if k_min <= ki <= n_i and k_min <= ko <= n_o:
                err = abs(ki * ko - k_total)
                if err < best_err:
                    best, best_err = (ki, ko), err
    ki, ko = best
    if ki < k_min or ko < k_min:
        raise ValueError(f"Cannot satisfy k_min={k_min} constraints with k_total={k_total}")
    return ki, ko


def _generator(seed: Optional[int]):
    if seed is None:
        return None
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def init_projection_matrix_gaussian(rows: int, cols: int, dtype: torch.dtype = torch.float32,
                                    device: torch.device = torch.device('cpu'),
                                    seed: Optional[int] = None) -> torch.Tensor:
    """[rows, cols] with entries N(0, 1/rows) (JL scaling, E[P^T P] = I)."""
    P = torch.randn(rows, cols, dtype=dtype, generator=_generator(seed)) * (1.0 / math.sqrt(rows))
    return P.to(device).requires_grad_(False)


def init_projection_matrix_rademacher(rows: int, cols: int, dtype: torch.dtype = torch.float32,
                                      device: torch.device = torch.device('cpu'),
                                      seed: Optional[int] = None) -> torch.Tensor:
    """[rows, cols] with entries +-1/sqrt(rows)."""
    signs = torch.randint(0, 2, (rows, cols), dtype=torch.int8, generator=_generator(seed))
    P = (signs * 2 - 1).to(dtype) * (1.0 / math.sqrt(rows))
    return P.to(device).requires_grad_(False)


def init_projection_matrix_orthonormal(rows: int, cols: int, dtype: torch.dtype = torch.float32,
                                       device: torch.device = torch.device('cpu'),
                                       seed: Optional[int] = None) -> torch.Tensor:
    """[rows, cols] with orthonormal rows (economy QR of a [cols, rows] Gaussian)."""
    if rows > cols:
        raise ValueError(f"Cannot create {rows} orthonormal rows in {cols} dimensions")
    M = torch.randn(cols, rows, dtype=torch.float64, generator=_generator(seed))
    Q, _ = torch.linalg.qr(M, mode='reduced')
    return Q.t().to(dtype).to(device).requires_grad_(False)


def get_projection_initializer(method: str = 'gaussian'):
    initializers = {
        'gaussian': init_projection_matrix_gaussian,
        'rademacher': init_projection_matrix_rademacher,
        'orthonormal': init_projection_matrix_orthonormal,
    }
    if method not in initializers:
        raise ValueError(f"Unknown projection method: {method}. "
                         f"Choose from {list(initializers.keys())}")
    return initializers[method]


def compute_projection_metadata(layer_name: str, layer: nn.Module, k_i: int, k_o: int) -> dict:
    """Per-layer metadata record (reference projection_utils.py:202-238)."""
    meta = {'name': layer_name, 'type': layer.__class__.__name__, 'k_i': k_i, 'k_o': k_o,
            'k_total': k_i * k_o}
    if isinstance(layer, nn.Embedding):
        meta['vocab_size'] = layer.num_embeddings
        meta['n_i'] = layer.num_embeddings
        meta['n_o'] = layer.embedding_dim
    elif hasattr(layer, 'weight'):
        ws = layer.weight.shape
        if isinstance(layer, nn.Linear):
            meta['n_o'], meta['n_i'] = ws
        elif isinstance(layer, nn.Conv1d):
            meta['n_o'] = ws[0]
            meta['n_i'] = ws[1] * ws[2]
        elif layer.__class__.__name__ == 'Conv1D':
            meta['n_o'], meta['n_i'] = ws
    return meta
