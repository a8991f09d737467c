"""Restatement of the reference samplers' arithmetic on the CPU (test infrastructure only).

Two flavours per sampler:
  *_ref    -- the reference's op sequence on torch CPU with its bf16 casts and rounding
              points (torch bf16 matmul/mul/sum round their outputs to bf16).
  *_exact  -- the same quantity in float64 with the casts removed (the "fp32 mode"
              authority and the closed form the brute-force tests check).
Layout follows the reference: rows [0, n_train) are train, the last n_val rows are val,
unless a function takes ``val_start``.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16


# ------------------------------------------------------------------ helpers
def split_rows(x: torch.Tensor, n_val: int, val_start: Optional[int] = None):
    """(train rows, val rows) for a val block at val_start (reference: val last)."""
    N = x.shape[0]
    vs = N - n_val if val_start is None else val_start
    val = x[vs:vs + n_val]
    train = torch.cat([x[:vs], x[vs + n_val:]], dim=0)
    return train, val


def tokens(A: torch.Tensor) -> int:
    """T as the reference computes it (supported_layers_grad_samplers_dotprod.py:26-29)."""
    return int(math.prod(A.shape[1:-1])) if A.dim() > 2 else 1


def should_use_ghost(T: int, weight_numel: int) -> bool:
    """The switch rule 2*T^2 <= weight.numel() (supported_layers_grad_samplers_dotprod.py:41)."""
    return bool(2 * T ** 2 <= weight_numel)


# ------------------------------------------------------------------ Linear
def linear_dot_ref(A: torch.Tensor, B: torch.Tensor, n_val: int, use_ghost: bool,
                   has_bias: bool = True) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """_compute_linear_dot_product (supported_layers_grad_samplers_dotprod.py:75-146).

    Ghost branch: bf16 casts (:92-93), two bf16 Gram matmuls (:125-126), bf16 Hadamard,
    fp32 sum over val tokens then over t (:129-130).  Materialised branch: original dtype,
    presum over val (:133-135).  Bias: original dtype (:137-146).
    """
    total = A.shape[0]
    n_t = total - n_val
    if n_t <= 0:
        raise ValueError("No training samples to compute dot product, check batch sizes.")
    A_tr_full, A_val_full = torch.split(A, [n_t, n_val], dim=0)
    B_tr_full, B_val_full = torch.split(B, [n_t, n_val], dim=0)
    if use_ghost:
        d, p = A.shape[-1], B.shape[-1]
        Ab, Bb = A.to(BF16), B.to(BF16)
        T = int(Ab.numel() // (total * d))
        Ab = Ab.reshape(total, T, d)
        Bb = Bb.reshape(total, T, p)
        a_tr = Ab[:n_t].reshape(-1, d).contiguous()
        a_va = Ab[n_t:].reshape(-1, d).contiguous()
        b_tr = Bb[:n_t].reshape(-1, p).contiguous()
        b_va = Bb[n_t:].reshape(-1, p).contiguous()
        a_dot = torch.matmul(a_tr, a_va.T)
        b_dot = torch.matmul(b_tr, b_va.T)
        tok = (a_dot * b_dot).sum(dim=1, dtype=torch.float32)
        w = tok.reshape(n_t, T).sum(dim=1)
    else:
        g_tr = torch.einsum('b...d,b...p->bpd', A_tr_full, B_tr_full)
        g_va = torch.einsum('...d,...p->dp', A_val_full.sum(dim=0), B_val_full.sum(dim=0))
        w = torch.einsum('dp,bpd->b', g_va, g_tr)
    b = None
    if has_bias:
        bv = B_val_full.sum(dim=list(range(B_val_full.dim() - 1)))
        bt = B_tr_full.sum(dim=list(range(1, B_tr_full.dim() - 1))) if B_tr_full.dim() > 2 \
            else B_tr_full
        b = torch.einsum('p,bp->b', bv, bt)
    return w, b


def linear_pair_ref(A: torch.Tensor, B: torch.Tensor, n_val: int) -> torch.Tensor:
    """Per-pair extension of the ghost branch: [n_val, n_train], entry (j, i) is the ghost
    sum restricted to val row j (the reference sums over j, :129)."""
    total = A.shape[0]
    n_t = total - n_val
    d, p = A.shape[-1], B.shape[-1]
    T = int(A.numel() // (total * d))
    Ab = A.to(BF16).reshape(total, T, d)
    Bb = B.to(BF16).reshape(total, T, p)
    a_tr = Ab[:n_t].reshape(-1, d)
    b_tr = Bb[:n_t].reshape(-1, p)
    out = torch.empty(n_val, n_t)
    for j in range(n_val):
        a_dot = torch.matmul(a_tr, Ab[n_t + j].T)
        b_dot = torch.matmul(b_tr, Bb[n_t + j].T)
        out[j] = (a_dot * b_dot).sum(dim=1, dtype=torch.float32).reshape(n_t, T).sum(dim=1)
    return out


def val_term_exact(A: torch.Tensor, B: torch.Tensor, n_val: int, semantics: str = "pairwise",
                   val_start: Optional[int] = None) -> torch.Tensor:
    """The val term V [d_out, d_in] (float64) the two semantics dot the train gradients with:
    pairwise sum_j G_j (the summed per-sample val gradients), presum (sum_j b_j)^T (sum_j a_j)
    (the materialised branch sums the val activations and backprops over the val samples
    per token position before the product, supported_layers_grad_samplers_dotprod.py:108-135).
    """
    N = A.shape[0]
    d, p = A.shape[-1], B.shape[-1]
    _, va_a = split_rows(A.double().reshape(N, -1, d), n_val, val_start)
    _, va_b = split_rows(B.double().reshape(N, -1, p), n_val, val_start)
    if semantics == "pairwise":
        return torch.einsum('ntp,ntd->pd', va_b, va_a)
    if semantics == "presum":
        return torch.einsum('tp,td->pd', va_b.sum(0), va_a.sum(0))
    raise ValueError(semantics)


def linear_dot_exact(A: torch.Tensor, B: torch.Tensor, n_val: int, semantics: str = "pairwise",
                     val_start: Optional[int] = None, pair: bool = False):
    """Float64 closed forms.

    pairwise: dot_i = <G_i, sum_j G_j>_F          (== ghost branch without casts)
    presum:   dot_i = <G_i, (sum_j b_j)^T (sum_j a_j)>  (== materialised branch, Conv1D)
    pair=True (pairwise only) returns [n_val, n_train] with entries <G_i, G_j>.
    """
    N = A.shape[0]
    d, p = A.shape[-1], B.shape[-1]
    tr_a, va_a = split_rows(A.double().reshape(N, -1, d), n_val, val_start)
    tr_b, va_b = split_rows(B.double().reshape(N, -1, p), n_val, val_start)
    G_tr = torch.einsum('ntp,ntd->npd', tr_b, tr_a)
    if semantics == "pairwise" and pair:
        G_va = torch.einsum('ntp,ntd->npd', va_b, va_a)
        return torch.einsum('ipd,jpd->ji', G_tr, G_va)
    if semantics == "presum" and pair:
        raise ValueError("presum has no per-pair form")
    return torch.einsum('ipd,pd->i', G_tr, val_term_exact(A, B, n_val, semantics, val_start))


def linear_dot_valterm_exact(A: torch.Tensor, B: torch.Tensor, n_val: int,
                             semantics: str = "pairwise",
                             val_start: Optional[int] = None,
                             round_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The linear_dot_exact vector through the val term: dot_i = sum_t b_it^T V a_it with V
    from val_term_exact, since <sum_t b_it a_it^T, V>_F = sum_t b_it^T V a_it.  Float64,
    with 2-D products only and one train row at a time, so that it runs at full model sizes
    on whichever device holds A and B (no [n_train, d_out, d_in] tensor is formed).

    ``round_dtype`` (e.g. bf16): the val-gradient kernels' rounding points, otherwise exact:
    the presummed val rows (presum) and V are rounded to that dtype before the products.  A
    dot whose train gradient is nearly orthogonal to V amplifies these roundings; this form
    then checks the kernels to their own arithmetic."""
    N = A.shape[0]
    d, p = A.shape[-1], B.shape[-1]
    a = A.reshape(N, -1, d)
    b = B.reshape(N, -1, p)
    vs = N - n_val if val_start is None else val_start
    va_a = a[vs:vs + n_val].double()
    va_b = b[vs:vs + n_val].double()
    rnd = (lambda x: x.to(round_dtype).double()) if round_dtype is not None else (lambda x: x)
    if semantics == "pairwise":
        V = torch.mm(va_b.reshape(-1, p).t(), va_a.reshape(-1, d))
    elif semantics == "presum":
        V = torch.mm(rnd(va_b.sum(0)).t(), rnd(va_a.sum(0)))
    else:
        raise ValueError(semantics)
    V = rnd(V)
    del va_a, va_b
    rows = [i for i in range(N) if not vs <= i < vs + n_val]
    out = torch.empty(len(rows), dtype=torch.float64, device=A.device)
    for k, i in enumerate(rows):
        out[k] = (torch.mm(b[i].double(), V) * a[i].double()).sum()
    return out


def bias_dot_exact(B: torch.Tensor, n_val: int, val_start: Optional[int] = None) -> torch.Tensor:
    N, p = B.shape[0], B.shape[-1]
    tr, va = split_rows(B.double().reshape(N, -1, p), n_val, val_start)
    return tr.sum(1) @ va.sum((0, 1))


def linear_train_grad(A: torch.Tensor, Bp: torch.Tensor, n_val: int) -> torch.Tensor:
    """_compute_linear_train_grad (supported_layers_grad_samplers_dotprod.py:155-173):
    sum over train rows of Bp^T A, divided by n_train (Bp are the N-scaled backprops)."""
    n_t = A.shape[0] - n_val
    A_tr, _ = torch.split(A, [n_t, n_val], dim=0)
    B_tr, _ = torch.split(Bp, [n_t, n_val], dim=0)
    g = torch.einsum('b...p,b...d->pd', B_tr, A_tr)
    g /= n_t
    return g


def bias_train_grad(Bp: torch.Tensor, n_val: int, loss_reduction: str = 'mean') -> torch.Tensor:
    """_compute_train_grad_bias (autograd_grad_sample_dotprod.py:199-222)."""
    n_t = Bp.size(0) - n_val
    if n_t <= 0:
        raise ValueError("No training samples to compute gradients, check batch sizes.")
    B_tr, _ = torch.split(Bp, [n_t, n_val], dim=0)
    s = B_tr.sum(dim=list(range(B_tr.dim() - 1)))
    if loss_reduction == 'mean':
        s /= n_t
    return s


# ------------------------------------------------------------------ Embedding
def embedding_dot_ref(ids: torch.Tensor, B: torch.Tensor, n_val: int, vocab: int) -> torch.Tensor:
    """_compute_embedding_dot_product (supported_layers_grad_samplers_dotprod.py:181-211):
    bf16 table by index_add_ of val rows (:203-208), bf16 gather-product, fp32 sum (:210)."""
    Bb = B.to(BF16)
    n_t = ids.size(0) - n_val
    if n_t <= 0:
        raise ValueError("No training samples to compute dot product, check batch sizes.")
    A_tr, A_va = torch.split(ids, [n_t, n_val], dim=0)
    B_tr, B_va = torch.split(Bb, [n_t, n_val], dim=0)
    d = B.shape[-1]
    table = torch.zeros((vocab, d), dtype=BF16)
    table.index_add_(0, A_va.long().reshape(-1), B_va.reshape(-1, d))
    return (B_tr * table[A_tr.long()]).float().sum(dim=[1, 2])


def embedding_dot_exact(ids: torch.Tensor, B: torch.Tensor, n_val: int,
                        val_start: Optional[int] = None) -> torch.Tensor:
    """sum_t <b_it, sum_{j,s: x_js = x_it} b_js> in float64 via the id-equality mask
    (the "mask times G Gram" form)."""
    N, d = B.shape[0], B.shape[-1]
    tr_i, va_i = split_rows(ids.reshape(N, -1).long(), n_val, val_start)
    tr_b, va_b = split_rows(B.double().reshape(N, -1, d), n_val, val_start)
    n_t = tr_i.shape[0]
    vi = va_i.reshape(-1)
    vb = va_b.reshape(-1, d)
    out = torch.empty(n_t, dtype=torch.float64, device=B.device)
    for i in range(n_t):
        mask = (tr_i[i][:, None] == vi[None, :]).double()       # [T, n_val*T]
        gram = tr_b[i] @ vb.T                                     # [T, n_val*T]
        out[i] = (mask * gram).sum()
    return out


def embedding_train_grad(ids: torch.Tensor, Bp: torch.Tensor, n_val: int,
                         weight_shape) -> torch.Tensor:
    """_compute_embedding_train_grad (supported_layers_grad_samplers_dotprod.py:214-235)."""
    n_t = ids.size(0) - n_val
    A_tr, _ = torch.split(ids, [n_t, n_val], dim=0)
    B_tr, _ = torch.split(Bp, [n_t, n_val], dim=0)
    g = torch.zeros(weight_shape, dtype=Bp.dtype)
    g.index_add_(0, A_tr.long().reshape(-1), B_tr.reshape(-1, B_tr.shape[-1]))
    g /= n_t
    return g


# ------------------------------------------------------------------ LayerNorm
def layernorm_dot_ref(A: torch.Tensor, B: torch.Tensor, n_val: int, eps: float,
                      has_bias: bool = True):
    """_compute_layernorm_dot_product (supported_layers_grad_samplers_dotprod.py:242-300):
    bf16 casts (:254-255), layer_norm without affine in bf16 (:262-263), bf16 products and
    per-sample sums, fp32 einsum (:281-283, :298-300)."""
    Ab, Bb = A.to(BF16), B.to(BF16)
    n_t = Ab.size(0) - n_val
    A_tr, A_va = torch.split(Ab, [n_t, n_val], dim=0)
    B_tr, B_va = torch.split(Bb, [n_t, n_val], dim=0)
    shape = (A.shape[-1],)
    na_tr = F.layer_norm(A_tr, shape, eps=eps)
    na_va = F.layer_norm(A_va, shape, eps=eps)
    gw_tr = B_tr * na_tr
    gw_va = B_va * na_va
    sd = list(range(1, gw_tr.dim() - 1))
    ps_w = gw_tr.sum(dim=sd) if sd else gw_tr
    tv_w = gw_va.sum(dim=list(range(gw_va.dim() - 1)))
    w = torch.einsum('bf,f->b', ps_w.float(), tv_w.float())
    b = None
    if has_bias:
        sd = list(range(1, B_tr.dim() - 1))
        ps_b = B_tr.sum(dim=sd) if sd else B_tr
        tv_b = B_va.sum(dim=list(range(B_va.dim() - 1)))
        b = torch.einsum('bf,f->b', ps_b.float(), tv_b.float())
    return w, b


def layernorm_dot_exact(A: torch.Tensor, B: torch.Tensor, n_val: int, eps: float,
                        val_start: Optional[int] = None):
    N, Fd = A.shape[0], A.shape[-1]
    x = A.double().reshape(N, -1, Fd)
    g = B.double().reshape(N, -1, Fd)
    xh = F.layer_norm(x, (Fd,), eps=eps)
    w = (g * xh).sum(1)
    b = g.sum(1)
    w_tr, w_va = split_rows(w, n_val, val_start)
    b_tr, b_va = split_rows(b, n_val, val_start)
    return w_tr @ w_va.sum(0), b_tr @ b_va.sum(0)


def layernorm_train_grad(A: torch.Tensor, Bp: torch.Tensor, n_val: int, eps: float,
                         has_bias: bool = True):
    """_compute_layernorm_train_grad (supported_layers_grad_samplers_dotprod.py:303-366)."""
    n_t = A.size(0) - n_val
    A_tr, _ = torch.split(A, [n_t, n_val], dim=0)
    B_tr, _ = torch.split(Bp, [n_t, n_val], dim=0)
    xh = F.layer_norm(A_tr, (A.shape[-1],), eps=eps)
    gw = (B_tr * xh).sum(dim=list(range(A_tr.dim() - 1)))
    gw /= n_t
    gb = None
    if has_bias:
        gb = B_tr.sum(dim=list(range(B_tr.dim() - 1)))
        gb /= n_t
    return gw, gb


# ------------------------------------------------------------------ HF Conv1D
def conv1d_dot_ref(A: torch.Tensor, B: torch.Tensor, n_val: int, use_ghost: bool,
                   has_bias: bool = True):
    """_compute_Conv1D_dot_product (supported_layers_grad_samplers_dotprod.py:369-471):
    presum semantics in both branches, all bf16."""
    Ab, Bb = A.to(BF16), B.to(BF16)
    n_t = Ab.size(0) - n_val
    A_tr, A_va = torch.split(Ab, [n_t, n_val], dim=0)
    B_tr, B_va = torch.split(Bb, [n_t, n_val], dim=0)
    if use_ghost:
        AA = torch.matmul(A_va.sum(0).unsqueeze(0), A_tr.transpose(-1, -2))
        BB = torch.matmul(B_va.sum(0).unsqueeze(0), B_tr.transpose(-1, -2))
        w = torch.sum((AA * BB).float(), dim=[1, 2])
    else:
        g_tr = torch.einsum('b...d, b...p->bpd', A_tr, B_tr)
        g_va = torch.einsum('...d, ...p->pd', A_va.sum(0), B_va.sum(0))
        w = torch.einsum('pd,bpd->b', g_va, g_tr)
    b = None
    if has_bias:
        bv = B_va.sum(dim=list(range(B_va.dim() - 1)))
        bt = B_tr.sum(dim=list(range(1, B_tr.dim() - 1)))
        b = torch.einsum('p,bp->b', bv, bt)
    return w, b


def conv2d_dot_ref(A: torch.Tensor, B: torch.Tensor, n_val: int, conv: dict,
                   has_bias: bool = True):
    """_compute_conv2d_dot_product, materialised branch (supported_layers_grad_samplers_dotprod.py
    :513-560): bf16 unfold, per-sample grads einsum('bik,bpk->bpi'), the val presum grad
    einsum('ik,pk->pi') of the val sums, then their dot; bias <sum_l b_il, sum_{j,l} b_jl>.
    (The reference's ghost branch multiplies [d,d] by [p,p] blocks and is not restated.)"""
    Ab, Bb = A.to(BF16), B.to(BF16)
    n_t = Ab.size(0) - n_val
    A_tr, A_va = torch.split(Ab, [n_t, n_val], dim=0)
    B_tr, B_va = torch.split(Bb, [n_t, n_val], dim=0)
    A_tr_u, A_va_u = F.unfold(A_tr, **conv), F.unfold(A_va, **conv)
    B_tr_r = B_tr.reshape(n_t, B_tr.size(1), -1)
    B_va_r = B_va.reshape(n_val, B_va.size(1), -1)
    g_tr = torch.einsum('bik,bpk->bpi', A_tr_u, B_tr_r)
    g_va = torch.einsum('ik,pk->pi', A_va_u.sum(dim=0), B_va_r.sum(dim=0))
    w = torch.einsum('pi,bpi->b', g_va, g_tr)
    b = None
    if has_bias:
        b = torch.einsum('p,bp->b', B_va_r.sum(dim=[0, 2]), B_tr_r.sum(dim=2))
    return w.float(), None if b is None else b.float()


def conv2d_ghost_ref(A: torch.Tensor, B: torch.Tensor, n_val: int, conv: dict) -> torch.Tensor:
    """_compute_conv2d_dot_product, ghost branch (supported_layers_grad_samplers_dotprod.py
    :546-550): bf16 unfold A_u [b, i, L] and B_r [b, p, L], the val sums over samples,
    AA = A_val_sum @ A_u^T ([b, i, i]) and BB = B_val_sum @ B_r^T ([b, p, p]), both bf16
    matmul outputs, then sum((AA * BB).float()) per train sample.  Defined when i == p."""
    Ab, Bb = A.to(BF16), B.to(BF16)
    n_t = Ab.size(0) - n_val
    A_tr, A_va = torch.split(Ab, [n_t, n_val], dim=0)
    B_tr, B_va = torch.split(Bb, [n_t, n_val], dim=0)
    A_tr_u, A_va_u = F.unfold(A_tr, **conv), F.unfold(A_va, **conv)
    B_tr_r = B_tr.reshape(n_t, B_tr.size(1), -1)
    B_va_r = B_va.reshape(n_val, B_va.size(1), -1)
    AA = torch.matmul(torch.sum(A_va_u, dim=0).unsqueeze(0), A_tr_u.transpose(1, 2))
    BB = torch.matmul(torch.sum(B_va_r, dim=0).unsqueeze(0), B_tr_r.transpose(1, 2))
    return torch.sum((AA * BB).float(), dim=[1, 2])


def conv2d_ghost_exact(A: torch.Tensor, B: torch.Tensor, n_val: int, conv: dict) -> torch.Tensor:
    """float64 value of the reference's Conv2d ghost-branch quantity, contracted in the other
    order: sum_{x,y} (Abar A_b^T)[x,y] (Bbar B_b^T)[x,y] = <Abar^T Bbar, A_b^T B_b> over
    [L, L] position pairs (Abar, Bbar the val sums of the unfolded A and of B)."""
    A64, B64 = A.double(), B.double()
    n_t = A64.size(0) - n_val
    A_u = F.unfold(A64, **conv)                            # [N, i, L]
    B_r = B64.reshape(B64.size(0), B64.size(1), -1)        # [N, p, L]
    cross_val = A_u[n_t:].sum(0).t() @ B_r[n_t:].sum(0)    # [L, L]
    cross_tr = torch.einsum('bxk,bxl->bkl', A_u[:n_t], B_r[:n_t])
    return torch.einsum('kl,bkl->b', cross_val, cross_tr)


def conv2d_dot_exact(A: torch.Tensor, B: torch.Tensor, n_val: int, conv: dict):
    """float64 presum dot of the Conv2d weight gradients: G_i = sum_l b_il a_il^T over the
    unfolded positions, Gbar the same with the val sums of a and b."""
    A64, B64 = A.double(), B.double()
    n_t = A64.size(0) - n_val
    A_u = F.unfold(A64, **conv)                            # [N, d, L]
    B_r = B64.reshape(B64.size(0), B64.size(1), -1)        # [N, p, L]
    G = torch.einsum('bdl,bpl->bpd', A_u[:n_t], B_r[:n_t])
    Gbar = torch.einsum('dl,pl->pd', A_u[n_t:].sum(0), B_r[n_t:].sum(0))
    return torch.einsum('bpd,pd->b', G, Gbar)


# ------------------------------------------------------------------ GradProj
def flatten_tokens(x: torch.Tensor) -> torch.Tensor:
    """_flatten_tokens (autograd_gradproj.py:11-37): [B, T, D]."""
    if x.dim() <= 2:
        return x.unsqueeze(1)
    return x.reshape(x.shape[0], -1, x.shape[-1])


def kron_proj_ref(A: torch.Tensor, B: torch.Tensor, P_i: torch.Tensor, P_o: torch.Tensor,
                  conv1d: bool = False) -> torch.Tensor:
    """_compute_dense_proj (autograd_gradproj.py:120-165), fp32 result."""
    A3 = flatten_tokens(A)
    B3 = flatten_tokens(B)
    bs = A3.shape[0]
    if conv1d:
        A_proj = torch.matmul(B3, P_i.t())
        B_proj = torch.matmul(A3, P_o.t())
        g = torch.einsum('bti,btj->bji', B_proj, A_proj)
    else:
        A_proj = torch.matmul(A3, P_i.t())
        B_proj = torch.matmul(B3, P_o.t())
        g = torch.einsum('bti,btj->bij', B_proj, A_proj)
    return (g * bs).to(torch.float32)


def kron_proj_exact(A: torch.Tensor, B: torch.Tensor, P_i: torch.Tensor, P_o: torch.Tensor,
                    scale: float, conv1d: bool = False) -> torch.Tensor:
    """scale * P_o G_b P_i^T per sample with G_b = sum_t b a^T, in float64 (the Kronecker
    identity vec(P_o G P_i^T) = (P_i (x) P_o) vec(G))."""
    A3 = flatten_tokens(A).double()
    B3 = flatten_tokens(B).double()
    Gs = torch.einsum('btp,btd->bpd', B3, A3)          # [B, n_out, n_in]
    if conv1d:
        # Conv1D: rows of P_i act on the output-grad side, P_o on the input side.
        return scale * torch.einsum('ip,bpd,od->bio', P_i.double(), Gs, P_o.double())
    return scale * torch.einsum('op,bpd,id->boi', P_o.double(), Gs, P_i.double())


def kron_proj_projfirst_exact(A: torch.Tensor, B: torch.Tensor, P_i: torch.Tensor,
                              P_o: torch.Tensor, scale: float,
                              conv1d: bool = False) -> torch.Tensor:
    """kron_proj_exact with the projections applied first: per sample
    scale * (B_b P_o^T)^T (A_b P_i^T) = scale * P_o (sum_t b a^T) P_i^T (Conv1D: P_i on the
    output-grad side, [k_i, k_o]).  Float64, 2-D products one sample at a time, so that it
    runs at full model sizes on whichever device holds A and B."""
    A3 = flatten_tokens(A)
    B3 = flatten_tokens(B)
    Pl, Pr = (P_i, P_o) if conv1d else (P_o, P_i)
    Pl = Pl.double().to(A3.device)
    Pr = Pr.double().to(A3.device)
    outs = []
    for b in range(A3.shape[0]):
        left = torch.mm(B3[b].double(), Pl.t())     # [T, k_o] (Conv1D: [T, k_i])
        right = torch.mm(A3[b].double(), Pr.t())    # [T, k_i] (Conv1D: [T, k_o])
        outs.append(scale * torch.mm(left.t(), right))
    return torch.stack(outs)


def kron_embed_proj_ref(ids: torch.Tensor, g: torch.Tensor, P_i: torch.Tensor,
                        P_o: torch.Tensor) -> torch.Tensor:
    """_compute_embedding_proj (autograd_gradproj.py:167-222): per sample, per token,
    accumulate (P_o g_t) (P_i[:, x_t])^T into a [k_o, k_i] fp32 matrix.  No batch-size
    factor (unlike the dense path).  A direct loop: small inputs only."""
    bs = ids.shape[0]
    ids2 = ids.reshape(bs, -1)
    g3 = g.reshape(bs, ids2.shape[1], g.shape[-1])
    out = []
    for b in range(bs):
        acc = torch.zeros(P_o.shape[0], P_i.shape[0], dtype=torch.float32)
        for t in range(ids2.shape[1]):
            j = int(ids2[b, t])
            acc += (P_o @ g3[b, t]).unsqueeze(1) @ P_i[:, j].unsqueeze(0)
        out.append(acc)
    return torch.stack(out).to(torch.float32)


def kron_embed_proj_exact(ids: torch.Tensor, g: torch.Tensor, P_i: torch.Tensor,
                          P_o: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """scale * P_o W_b P_i^T in float64, where W_b = sum_t g_t e_{x_t}^T is sample b's
    embedding-weight gradient (transposed to [d, vocab])."""
    bs = ids.shape[0]
    ids2 = ids.reshape(bs, -1).long()
    g3 = g.reshape(bs, ids2.shape[1], g.shape[-1]).double()
    W = torch.zeros(bs, g3.shape[-1], P_i.shape[1], dtype=torch.float64)
    W.scatter_add_(2, ids2.unsqueeze(1).expand(bs, g3.shape[-1], ids2.shape[1]),
                   g3.transpose(1, 2))
    return scale * torch.einsum('od,bdv,iv->boi', P_o.double(), W, P_i.double())


def kron_embed_proj_projfirst_exact(ids: torch.Tensor, g: torch.Tensor, P_i: torch.Tensor,
                                    P_o: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """kron_embed_proj_exact with the projections applied first: per sample
    scale * (G_b P_o^T)^T P_i[:, ids_b]^T.  Float64, 2-D products one sample at a time, on
    whichever device holds g (no [vocab]-wide per-sample gradient is formed)."""
    bs = ids.shape[0]
    ids2 = ids.reshape(bs, -1).long()
    g3 = g.reshape(bs, ids2.shape[1], g.shape[-1])
    P_iT = P_i.double().to(g3.device).t()
    P_o = P_o.double().to(g3.device)
    outs = []
    for b in range(bs):
        left = torch.mm(g3[b].double(), P_o.t())      # [T, k_o]
        right = P_iT[ids2[b].to(g3.device)]           # [T, k_i]
        outs.append(scale * torch.mm(left.t(), right))
    return torch.stack(outs)


def choose_ki_ko(n_i: int, n_o: int, k_total: int, k_min: int = 1):
    """choose_ki_ko (projection_utils.py:12-66): ratio rule, then a +-2 search with
    strict-improvement tie-break."""
    if min(n_i, n_o) <= 0 or k_total <= 0:
        raise ValueError(f"Invalid dimensions for projection: n_i={n_i}, n_o={n_o}, k_total={k_total}")
    if k_min > min(n_i, n_o):
        raise ValueError(f"k_min={k_min} exceeds layer dimensions (n_i={n_i}, n_o={n_o})")
    root = math.sqrt(k_total)
    r = math.sqrt(n_o / max(1, n_i))
    k_i = max(k_min, min(n_i, max(1, int(round(root * r)))))
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


# ------------------------------------------------------------------ tolerances
def normwise_close(x: torch.Tensor, y: torch.Tensor, tol: float) -> Tuple[bool, float]:
    """|x - y| <= tol * max(|y|, rms(y)) elementwise (near-zero entries of a sum with
    cancellation are judged against the vector's scale).  Returns (ok, worst ratio)."""
    x = x.double().cpu().reshape(-1)
    y = y.double().cpu().reshape(-1)
    if x.shape != y.shape:
        return False, float("inf")
    if y.numel() == 0:
        return True, 0.0
    rms = y.pow(2).mean().sqrt().item()
    scale = torch.clamp(y.abs(), min=max(rms, 1e-300))
    worst = ((x - y).abs() / scale).max().item()
    return worst <= tol, worst
