"""Per-layer samplers of the GradDotProd engine, backed by the gfx950 kernels.

Same registry, function names, signatures, side effects and exceptions as the reference
(ghostEngines/supported_layers_grad_samplers_dotprod.py); the arithmetic runs in
libghost_hip.so (one C-ABI call per sampler, asynchronous on the current stream).

Semantics kept from the reference:
  - the ghost/materialise switch 2*T^2 <= weight.numel(), cached on the layer (:7-41);
  - nn.Linear: ghost branch = pairwise-sum over val rows, materialised branch = presum
    (:108-135); HF Conv1D: presum in both branches (:369-447);
  - bias dots <sum_t b_it, sum_{j,t} b_jt> (:137-146);
  - embedding dot through token-id equality (:181-211), LayerNorm weight/bias dots (:242-300);
  - train gradients averaged over the train rows of the N-scaled backprops, accumulated
    into ``param.train_grad`` (:44-69).
Algorithm choice inside a semantics is this build's (``options['linear_algo']``): the fused
ghost kernel or the val-gradient form, by MFMA flop count when 'auto'.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from . import _native, _overlap
from ._native import ops

try:  # HF Conv1D is a registry key only when transformers is importable
    import transformers.pytorch_utils as _hf_utils
    _HFConv1D = _hf_utils.Conv1D
except Exception:  # pragma: no cover - transformers absent
    _HFConv1D = None

# Engine-wide knobs.  Each GradDotProdEngine resets them to DEFAULT_OPTIONS and applies its
# keyword arguments; they can also be changed directly between steps.
#   precision:     'reference' -- bf16 operands for the ghost/pairwise path (the reference
#                  casts A, B to bf16, :92-93), original dtype for presum (:104-105);
#                  'fp32' -- no down-casts (fp32 operands everywhere).
#   linear_algo:   'auto' | 'ghost' | 'valgrad'
#   rounding:      'fp32' | 'ref_bf16' (ghost Gram entries rounded to bf16 like the
#                  reference's bf16 matmul outputs)
#   store_pairs:   also keep the [n_val, n_train] per-pair matrix on pairwise-sum Linear
#                  layers as ``weight.grad_dot_prod_pair``
#   skip_overwritten_tied_dots: skip a tied Linear weight's dot when the Embedding that
#                  shares the weight runs later in backward and overwrites it (:130 vs :211)
#   record_algorithms: keep {layer name: algorithm} in ``ALGO_LOG``
#   reference_id_promotion: pass an Embedding's token ids through the backprops' dtype
#                  before its dot, as the reference's hook does (ids >= 256 round in a bf16
#                  model); off by default: the ids are used as given
#   reference_conv2d_ghost: a Conv2d layer on the reference's ghost branch gets that branch's
#                  quantity, sum over [i, i] of (the val-summed unfolded input Gram) times
#                  (the val-summed backprop Gram), i = C_in*kh*kw = C_out (:546-550), instead
#                  of the presum dot of the per-sample gradients that both branches aim at;
#                  off by default
#   dot_dtypes:    'reference' -- each grad_dot_prod in the dtype the reference's sampler
#                  returns: the materialised-branch weight dots and the bias dots of Linear,
#                  Conv1D and Conv2d layers in the operands' dtype (bf16 in a bf16 model),
#                  every other dot fp32; 'fp32' -- every dot fp32 (the kernels' own output)
options = {
    "precision": "reference",
    "linear_algo": "auto",
    "rounding": "fp32",
    "store_pairs": False,
    "skip_overwritten_tied_dots": True,
    "record_algorithms": False,
    # Run the dot kernels on a side stream, overlapped with the rest of backward.
    "overlap": True,
    "reference_id_promotion": False,
    "reference_conv2d_ghost": False,
    "dot_dtypes": "reference",
}
DEFAULT_OPTIONS = dict(options)
ALGO_LOG: dict = {}

_ALGOS = {"auto": _native.ALGO_AUTO, "ghost": _native.ALGO_GHOST, "valgrad": _native.ALGO_VALGRAD}
_ROUNDINGS = {"fp32": _native.ROUND_FP32, "ref_bf16": _native.ROUND_REF_BF16}


def _should_use_ghost_computation(layer: nn.Module, A: torch.Tensor, B: torch.Tensor,
                                  conv: bool = False):
    """Caches ``layer.use_ghost_computation = 2*T^2 <= weight.numel()`` on the first call
    (reference :7-41; never reset)."""
    if hasattr(layer, "use_ghost_computation"):
        return
    if not conv:
        T = math.prod(A.shape[1:-1]) if A.dim() > 2 else 1
    else:
        T = A.shape[-1]
    layer.use_ghost_computation = bool(2 * T ** 2 <= layer.weight.numel())


def _create_or_accumulate_train_grad(param: torch.Tensor, grad: torch.Tensor) -> None:
    """Stores or adds ``grad`` into ``param.train_grad`` (reference :44-69)."""
    assert grad.shape == param.shape, \
        f"Gradient shape ({grad.shape}) does not match parameter shape ({param.shape})"
    new_grad = grad.detach()
    if hasattr(param, 'train_grad'):
        _overlap.join(new_grad.device)   # either addend may come from the side stream
        param.train_grad.add_(new_grad)
    else:
        param.train_grad = new_grad


def _train_split(A: torch.Tensor, val_batch_size: int):
    n_t = A.size(0) - val_batch_size
    return n_t, A[:n_t]


def _dot_dtype(x: torch.Tensor, pairwise: bool) -> torch.dtype:
    if options["precision"] == "fp32":
        return torch.float32
    if pairwise:
        return torch.bfloat16
    return x.dtype if x.dtype in (torch.bfloat16, torch.float32) else torch.float32


def _reference_dtypes(layer: nn.Module, weight_dtype: Optional[torch.dtype],
                      bias_dtype: Optional[torch.dtype]) -> None:
    """Casts the dots the sampler set to the dtypes the reference's sampler returns (a None
    dtype: left fp32).  Its materialised branches and bias dots are einsums over operands in
    the layer's dtype (Linear :131-146 in the original dtype, Conv1D :445-471 and Conv2d
    :552-559 in bf16); its ghost branches sum in fp32 (:129-130, :437, :550)."""
    if options["dot_dtypes"] != "reference" or options["precision"] == "fp32":
        return
    for param, dt in ((layer.weight, weight_dtype), (getattr(layer, "bias", None), bias_dtype)):
        if param is None or dt is None:
            continue
        dot = param.__dict__.get("grad_dot_prod")
        if dot is not None and dot.dtype != dt:
            param.grad_dot_prod = dot.to(dt)


def _overwritten_later(layer: nn.Module) -> bool:
    """True when this Linear's weight is tied to a hooked Embedding whose forward ran
    earlier in the current step, so the Embedding's backward hook runs later and its
    assignment of ``grad_dot_prod`` replaces this layer's."""
    if not options["skip_overwritten_tied_dots"]:
        return False
    emb = getattr(layer, "_gs_tied_embedding", None)
    if emb is None:
        return False
    mine, theirs = getattr(layer, "_gs_fwd_seq", None), getattr(emb, "_gs_fwd_seq", None)
    return mine is not None and theirs is not None and theirs[0] == mine[0] and theirs[1] < mine[1]


def _bias_dot_and_grad(layer: nn.Module, B: torch.Tensor, val_batch_size: int,
                       dtype: torch.dtype) -> None:
    """Bias dot (reference :137-146); when the hook announced the train-grad scale, the
    same pass also produces the bias train gradient and parks it for _apply_train_grad."""
    scale = getattr(layer, "_gs_bias_grad_scale", None)
    dot, grad = ops().bias_dot(B.to(dtype) if B.dtype != dtype else B, val_batch_size,
                               grad_scale=scale, grad_dtype=layer.bias.dtype)
    layer.bias.grad_dot_prod = dot
    if grad is not None:
        layer._gs_bias_train_grad = grad


# Linear Layer ##############################################################################

def _linear_like_dot(layer: nn.Module, A: torch.Tensor, B: torch.Tensor, val_batch_size: int,
                     pairwise: bool, dtype: torch.dtype) -> None:
    if options["store_pairs"] and pairwise:
        want_pair = True
    else:
        want_pair = False
    Ac = A.to(dtype) if A.dtype != dtype else A
    Bc = B.to(dtype) if B.dtype != dtype else B
    sem = _native.SEM_PAIRWISE_SUM if pairwise else _native.SEM_PRESUM
    algo = _ALGOS[options["linear_algo"]]
    if options["record_algorithms"]:
        N, d_in, d_out = Ac.shape[0], Ac.shape[-1], Bc.shape[-1]
        T = Ac.numel() // (N * d_in)
        chosen = ops().linear_algo(dtype, N, val_batch_size, T, d_in, d_out, sem, algo,
                                   want_pair)
        ALGO_LOG[getattr(layer, "name", id(layer))] = (
            "pairwise" if pairwise else "presum", _native.ALGO_NAMES.get(chosen, str(chosen)))
    dot, pair = ops().linear_dot(Ac, Bc, val_batch_size, semantics=sem, algo=algo,
                                 rounding=_ROUNDINGS[options["rounding"]], want_pair=want_pair)
    layer.weight.grad_dot_prod = dot
    if pair is not None:
        layer.weight.grad_dot_prod_pair = pair


def _compute_linear_dot_product(layer: nn.Linear, A: torch.Tensor, B: torch.Tensor,
                                val_batch_size: int):
    """Gradient dot-product of an nn.Linear layer (reference :75-146).

    Sets ``layer.weight.grad_dot_prod`` ([n_train]) and, with a bias,
    ``layer.bias.grad_dot_prod``: fp32 from the ghost branch (pairwise sum), in the
    operands' dtype from the materialised branch and for the bias, as the reference returns
    them (``dot_dtypes='fp32'``: always fp32).
    """
    if A is None:
        raise ValueError("Input activations A cannot be None.")
    if B is None:
        raise ValueError("Output gradients B cannot be None.")
    A = A.detach()
    B = B.detach()
    train_bs = A.size(0) - val_batch_size
    if train_bs <= 0:
        raise ValueError("No training samples to compute dot product, check batch sizes.")
    _should_use_ghost_computation(layer, A, B)
    _linear_dots(layer, A, B, val_batch_size)
    _reference_dtypes(layer, None if layer.use_ghost_computation else A.dtype, B.dtype)


def _linear_dots(layer: nn.Linear, A: torch.Tensor, B: torch.Tensor, val_batch_size: int):
    pairwise = layer.use_ghost_computation
    if not _overwritten_later(layer):
        dt = _dot_dtype(A, pairwise)
        if _fused_dot_train_grad(layer, A, B, val_batch_size, pairwise, dt):
            return
        if layer.bias is not None and _fused_bias_dot(layer, A, B, val_batch_size, pairwise, dt,
                                                      _dot_dtype(B, False)):
            return
        _linear_like_dot(layer, A, B, val_batch_size, pairwise, dt)
    if layer.bias is not None:
        _bias_dot_and_grad(layer, B, val_batch_size, _dot_dtype(B, False))


def _fused_dot_train_grad(layer: nn.Module, A: torch.Tensor, B: torch.Tensor,
                          val_batch_size: int, pairwise: bool, dtype: torch.dtype,
                          conv1d: bool = False) -> bool:
    """Weight dot and weight train gradient (and with a bias its dot and train gradient) from
    one K-major pass over the train rows: per train row, sum_t g^T V a = <V, G_i^T A_i>, and
    the train gradient is the sum of the same G_i^T A_i (gs_linear_dot_train_grad).  Taken
    for bf16 layers on the val-gradient algorithm whose weight trains; the train gradients
    are parked for _apply_train_grad.  Returns False when the other paths must run.

    With ``conv1d`` (HF Conv1D, weight [d_in, d_out]) the Conv1D entry point runs the same
    pass with the operands swapped: the dot <G_i^T A_i, V> equals <A_i^T G_i, V^T>, the train
    gradient comes out as the sum of A_i^T G_i (the Conv1D layout), and the bias terms come
    from the column sums of G as for a Linear layer."""
    scale = getattr(layer, "_gs_bias_grad_scale", None)
    bias = layer.bias is not None
    grad_dtypes = (torch.bfloat16, torch.float32)   # train gradients in the parameters' dtype
    if scale is None or dtype != torch.bfloat16 or A.dtype != torch.bfloat16 or \
            (pairwise and options["store_pairs"]) or \
            layer.weight.dtype not in grad_dtypes or \
            not getattr(layer.weight, "initially_requires_grad", False) or \
            (bias and (layer.bias.dtype not in grad_dtypes or
                       not getattr(layer.bias, "initially_requires_grad", False))):
        return False
    Bc = B.to(dtype) if B.dtype != dtype else B
    N, d_in, d_out = A.shape[0], A.shape[-1], Bc.shape[-1]
    T = A.numel() // (N * d_in)
    sem = _native.SEM_PAIRWISE_SUM if pairwise else _native.SEM_PRESUM
    if ops().linear_algo(dtype, N, val_batch_size, T, d_in, d_out, sem,
                         _ALGOS[options["linear_algo"]], False) != _native.ALGO_VALGRAD:
        return False
    res = ops().linear_dot_train_grad(A, Bc, val_batch_size, semantics=sem, grad_scale=scale,
                                      grad_dtype=layer.weight.dtype, bias=bias,
                                      bias_grad_scale=scale,
                                      bias_grad_dtype=layer.bias.dtype if bias else None,
                                      conv1d=conv1d)
    if res is None:
        return False
    dot, grad, bias_dot, bias_grad = res
    layer.weight.grad_dot_prod = dot
    layer._gs_weight_train_grad = grad
    if bias:
        layer.bias.grad_dot_prod = bias_dot
        layer._gs_bias_train_grad = bias_grad
    if options["record_algorithms"]:
        ALGO_LOG[getattr(layer, "name", id(layer))] = ("pairwise" if pairwise else "presum",
                                                       "valgrad+train_grad")
    return True


def _fused_bias_dot(layer: nn.Module, A: torch.Tensor, B: torch.Tensor, val_batch_size: int,
                    pairwise: bool, dtype: torch.dtype, bias_dtype: torch.dtype) -> bool:
    """Weight dot, bias dot and bias train gradient from one pass over the train rows of B,
    when the kernel layer supports the shape (bf16 dots, val-gradient algorithm).  Returns
    False when the separate weight and bias passes must run instead."""
    if (pairwise and options["store_pairs"]) or dtype != torch.bfloat16 or \
            bias_dtype != torch.bfloat16:
        return False
    sem = _native.SEM_PAIRWISE_SUM if pairwise else _native.SEM_PRESUM
    fused = ops().linear_bias_dot(
        A.to(dtype), B.to(dtype), val_batch_size, semantics=sem,
        algo=_ALGOS[options["linear_algo"]], rounding=_ROUNDINGS[options["rounding"]],
        grad_scale=getattr(layer, "_gs_bias_grad_scale", None), grad_dtype=layer.bias.dtype)
    if fused is None:
        return False
    dot, bias_dot, bias_grad = fused
    layer.weight.grad_dot_prod = dot
    layer.bias.grad_dot_prod = bias_dot
    if bias_grad is not None:
        layer._gs_bias_train_grad = bias_grad
    if options["record_algorithms"]:
        ALGO_LOG[getattr(layer, "name", id(layer))] = ("pairwise" if pairwise else "presum",
                                                       "valgrad+bias")
    return True


def _compute_linear_train_grad(layer: nn.Linear, A: torch.Tensor, B: torch.Tensor,
                               val_batch_size: int, scale: float = 1.0):
    """scale * sum_train B^T A / n_train (reference :155-173, with B pre-scaled there;
    here the N-scaling of the backprops may be passed as ``scale``)."""
    n_t = A.size(0) - val_batch_size
    if n_t <= 0:
        return None
    parked = layer.__dict__.pop("_gs_weight_train_grad", None)
    if parked is not None:   # formed with the dots (_fused_dot_train_grad), same scale
        return parked
    wdt = _grad_dtype(layer, A)
    grad = _native_train_grad(A, B, val_batch_size, scale / n_t, False, wdt)
    if grad is not None:
        return grad
    A_tr = A[:n_t].reshape(-1, A.shape[-1])
    B_tr = B[:n_t].reshape(-1, B.shape[-1])
    if B_tr.dtype != A_tr.dtype:
        B_tr = B_tr.to(A_tr.dtype)
    return _scaled_mm(B_tr.t(), A_tr, scale / n_t).to(wdt)


def _grad_dtype(layer: nn.Module, A: torch.Tensor) -> torch.dtype:
    """The dtype a weight's train gradient is formed in: the parameter's own, so that it can
    become the parameter's .grad (under autocast the operands may be bf16 while the parameter
    is fp32), else the activations'."""
    wdt = layer.weight.dtype
    return wdt if wdt in (torch.bfloat16, torch.float32, torch.float16) else A.dtype


# Where the K-major train-gradient GEMM beats hipBLASLt (measured on MI355X, 16k-32k train
# token rows): below 256 output tiles of 128 x 128 it splits the long token contraction
# (GPT-2-small fc / fc_out 85-88 us against 152-160 us through torch.addmm, proj 31 against
# 98); from 256 tiles of 256 x 256 up its wide-tile kernel fills the chip without a split
# (Pythia-1B fc / fc_out 430-443 us against 505-511, embed_out 2851 against 3085); in between
# (e.g. 2048 x 6144: 470 against 354 us) hipBLASLt is faster.  The GPT-2 lm_head (50257
# columns) is not 16-byte aligned and takes hipBLASLt either way.
_TRAIN_GRAD_MAX_TILES = 256
_TRAIN_GRAD_WIDE_TILES = 256


def _native_train_grad(A: torch.Tensor, B: torch.Tensor, val_batch_size: int, alpha: float,
                       conv1d: bool, out_dtype: torch.dtype) -> Optional[torch.Tensor]:
    """The weight's train gradient from the K-major GEMM over the train rows as they lie
    (gs_linear_train_grad: fp32 accumulation, alpha before the one rounding to out_dtype);
    None where that kernel does not apply (fp32 operands or output dtype other than bf16 /
    fp32, unaligned or >2 GiB rows) or where hipBLASLt is faster (from _TRAIN_GRAD_MAX_TILES
    tiles of 128 x 128 to below _TRAIN_GRAD_WIDE_TILES tiles of 256 x 256)."""
    if A.dtype != torch.bfloat16 or A.dim() < 2 or \
            out_dtype not in (torch.bfloat16, torch.float32):
        return None
    tiles = math.ceil(A.shape[-1] / 128) * math.ceil(B.shape[-1] / 128)
    wide = math.ceil(A.shape[-1] / 256) * math.ceil(B.shape[-1] / 256)
    if _TRAIN_GRAD_MAX_TILES <= tiles and wide < _TRAIN_GRAD_WIDE_TILES:
        return None
    B = B if B.dtype == A.dtype else B.to(A.dtype)
    return ops().linear_train_grad(A, B, val_batch_size, alpha,
                                   val_start=A.size(0) - val_batch_size, out_dtype=out_dtype,
                                   conv1d=conv1d)


def _scaled_mm(x: torch.Tensor, y: torch.Tensor, alpha: float) -> torch.Tensor:
    """alpha * x @ y with alpha applied in the GEMM's fp32 epilogue: one rounding to the
    output dtype and no second pass over the result."""
    return torch.addmm(torch.zeros((), dtype=x.dtype, device=x.device), x, y, beta=0.0,
                       alpha=alpha)


# Embedding Layer ###########################################################################

def _compute_embedding_dot_product(layer: nn.Embedding, A: torch.Tensor, B: torch.Tensor,
                                   val_batch_size: int):
    """Gradient dot-product of an nn.Embedding (reference :181-211)."""
    A = A.detach()
    B = B.detach()
    train_bs = A.size(0) - val_batch_size
    if train_bs <= 0:
        raise ValueError("No training samples to compute dot product, check batch sizes.")
    if options["precision"] == "fp32" and B.dtype != torch.float32:
        B = B.float()
    elif B.dtype not in (torch.bfloat16, torch.float32):
        B = B.float()
    layer.weight.grad_dot_prod = ops().embedding_dot(A, B, val_batch_size,
                                                     vocab=layer.weight.shape[0])
    # With the train-grad scale announced, the train gradient is formed here as well (same
    # stream as the dot, no second hook-stage launch sequence) and parked for
    # _compute_embedding_train_grad.
    scale = getattr(layer, "_gs_bias_grad_scale", None)
    if scale is not None and getattr(layer.weight, "initially_requires_grad", False):
        # The train gradient is built from the ids the layer saw: the reference's gradient
        # stage reads layer.activations (autograd_grad_sample_dotprod.py:166-181), not the ids
        # its dot stage promoted to the backprops' dtype (:116-123), which may have rounded.
        ids = layer.__dict__.get("activations")
        ids = A if ids is None or ids.is_floating_point() else ids.detach()
        layer._gs_weight_train_grad = _embedding_train_grad(layer, ids, B, val_batch_size,
                                                            scale, join=False)


# Returned by a train-grad sampler that has already added its gradient into
# ``param.train_grad`` itself.
APPLIED = object()


def _compute_embedding_train_grad(layer: nn.Embedding, A: torch.Tensor, B: torch.Tensor,
                                  val_batch_size: int, scale: float = 1.0):
    """scale * (sum of the train rows per token id) / n_train (reference :214-235), summed
    in fp32 and rounded once to the weight dtype (the reference accumulates with index_add_
    in the weight dtype).  The kernel writes every row of a fresh gradient once (no
    zero-fill and full-table scale); when the weight already holds a train gradient (a tied
    lm_head's, computed earlier in backward) it adds the touched rows into that tensor and
    this returns APPLIED."""
    n_t = A.size(0) - val_batch_size
    if n_t <= 0:
        return None
    parked = layer.__dict__.pop("_gs_weight_train_grad", None)
    if parked is not None:   # formed with the dot, same scale
        return parked
    return _embedding_train_grad(layer, A, B, val_batch_size, scale / n_t, join=True)


def _embedding_train_grad(layer: nn.Embedding, A: torch.Tensor, B: torch.Tensor,
                          val_batch_size: int, alpha: float, join: bool):
    """alpha * (sum of the train rows of B per token id) as a fresh gradient, or added into
    the weight's existing train gradient (then APPLIED).  ``join``: order the current stream
    after the side stream first (not needed on the side stream itself)."""
    B = B.detach()
    if B.dtype not in (torch.bfloat16, torch.float32):
        B = B.float()
    prev = getattr(layer.weight, "train_grad", None)
    if prev is not None and prev.shape == layer.weight.shape:
        if join:
            _overlap.join(prev.device)   # prev may come from the side stream
        ops().embedding_train_grad(A.detach(), B, val_batch_size, alpha, prev, accumulate=True)
        return APPLIED
    grad = torch.empty_like(layer.weight)
    ops().embedding_train_grad(A.detach(), B, val_batch_size, alpha, grad)
    return grad


# LayerNorm Layer ###########################################################################

def _ln_features(layer: nn.LayerNorm) -> int:
    if len(layer.normalized_shape) != 1:
        raise NotImplementedError("LayerNorm over more than the last dimension is not supported")
    return layer.normalized_shape[0]


def _compute_layernorm_dot_product(layer: nn.LayerNorm, A: torch.Tensor, B: torch.Tensor,
                                   val_batch_size: int):
    """Weight/bias dot-products of an nn.LayerNorm (reference :242-300).  The same pass
    produces the train gradients when the hook announced their scale."""
    A = A.detach()
    B = B.detach()
    train_bs = A.size(0) - val_batch_size
    if train_bs <= 0:
        return
    _ln_features(layer)
    dt = torch.float32 if options["precision"] == "fp32" else (
        A.dtype if A.dtype in (torch.bfloat16, torch.float32) else torch.float32)
    Ac = A.to(dt) if A.dtype != dt else A
    Bc = B.to(dt) if B.dtype != dt else B
    scale = getattr(layer, "_gs_ln_grad_scale", None)
    dw, db, gw, gb = ops().layernorm_dot(
        Ac, Bc, val_batch_size, layer.eps, want_dot=True, want_bias=layer.bias is not None,
        grad_scale=scale, grad_dtype=layer.weight.dtype)
    layer.weight.grad_dot_prod = dw
    if layer.bias is not None:
        layer.bias.grad_dot_prod = db
    if gw is not None:
        layer._gs_ln_train_grads = (gw, gb)


def _compute_layernorm_train_grad(layer: nn.LayerNorm, A: torch.Tensor, B: torch.Tensor,
                                  val_batch_size: int, scale: float = 1.0) -> None:
    """Applies the LayerNorm train gradients itself and returns None (reference :303-366)."""
    train_bs = A.size(0) - val_batch_size
    if train_bs <= 0:
        raise ValueError("No training samples to compute gradients, check batch sizes.")
    stash = layer.__dict__.pop("_gs_ln_train_grads", None)
    if stash is None:
        _ln_features(layer)
        dt = A.dtype if A.dtype in (torch.bfloat16, torch.float32) else torch.float32
        _, _, gw, gb = ops().layernorm_dot(
            A.detach().to(dt), B.detach().to(dt), val_batch_size, layer.eps, want_dot=False,
            want_bias=layer.bias is not None, grad_scale=scale / train_bs,
            grad_dtype=layer.weight.dtype)
    else:
        gw, gb = stash
    _create_or_accumulate_train_grad(layer.weight, gw)
    if layer.bias is not None:
        _create_or_accumulate_train_grad(layer.bias, gb)
    return None


# HF Conv1D (weight [d_in, d_out]) ##########################################################

def _compute_Conv1D_dot_product(layer, A: torch.Tensor, B: torch.Tensor, val_batch_size: int):
    """Conv1D dot-products (reference :369-471): presum in both branches, bf16 operands; the
    ghost branch's dot fp32, the materialised branch's and the bias dot bf16, as the
    reference returns them (``dot_dtypes='fp32'``: always fp32)."""
    if A is None:
        raise ValueError("Input activations A cannot be None.")
    if B is None:
        raise ValueError("Output gradients B cannot be None.")
    A = A.detach()
    B = B.detach()
    train_bs = A.size(0) - val_batch_size
    if train_bs <= 0:
        raise ValueError("No training samples to compute dot product, check batch sizes.")
    _should_use_ghost_computation(layer, A, B)
    if A.dim() > 3:
        raise ValueError("Currently we only expect 3D input tensors (batch, seq_len, features). "
                         "Extending this to 4D or higher requires additional handling.")
    dt = torch.float32 if options["precision"] == "fp32" else torch.bfloat16
    if not _fused_dot_train_grad(layer, A, B, val_batch_size, False, dt, conv1d=True) and \
            not (layer.bias is not None and
                 _fused_bias_dot(layer, A, B, val_batch_size, False, dt, dt)):
        _linear_like_dot(layer, A, B, val_batch_size, False, dt)
        if layer.bias is not None:
            _bias_dot_and_grad(layer, B, val_batch_size, dt)
    _reference_dtypes(layer, None if layer.use_ghost_computation else torch.bfloat16,
                      torch.bfloat16)


def _compute_Conv1D_train_grad(layer, A: torch.Tensor, B: torch.Tensor, val_batch_size: int,
                               scale: float = 1.0) -> torch.Tensor:
    """scale * sum_train A^T B / n_train, [d_in, d_out] (reference :474-506)."""
    n_t = A.size(0) - val_batch_size
    parked = layer.__dict__.pop("_gs_weight_train_grad", None)
    if parked is not None:   # formed with the dots (_fused_dot_train_grad), same scale
        return parked
    wdt = _grad_dtype(layer, A)
    grad = _native_train_grad(A, B, val_batch_size, scale / n_t, True, wdt)
    if grad is not None:
        return grad
    A_tr = A[:n_t].reshape(-1, A.shape[-1])
    B_tr = B[:n_t].reshape(-1, B.shape[-1]).to(A_tr.dtype)
    return _scaled_mm(A_tr.t(), B_tr, scale / n_t).to(wdt)


# Conv2d ###################################################################################

def _conv2d_rows(layer: nn.Conv2d, A: torch.Tensor, B: torch.Tensor, dtype: torch.dtype):
    """im2col as token-major rows: A -> [N, L, C_in*kh*kw] (the unfold's feature order, which
    is the order of weight.view(C_out, -1)), B -> [N, L, C_out]; L = output positions."""
    if layer.groups != 1:
        raise NotImplementedError("Conv2d with groups > 1 is not supported")
    if isinstance(layer.padding, str):
        raise NotImplementedError("Conv2d with string padding is not supported")
    A_u = F.unfold(A.to(dtype), kernel_size=layer.kernel_size, dilation=layer.dilation,
                   padding=layer.padding, stride=layer.stride)
    A_rows = A_u.transpose(1, 2).contiguous()
    B_rows = B.to(dtype).reshape(B.size(0), B.size(1), -1).transpose(1, 2).contiguous()
    return A_rows, B_rows


def _conv2d_reference_ghost(layer: nn.Conv2d, A: torch.Tensor, B: torch.Tensor, n_val: int,
                            dtype: torch.dtype) -> torch.Tensor:
    """The reference's Conv2d ghost-branch quantity (:546-550): with the unfolded inputs
    A_u [N, i, L] and backprops B_r [N, p, L], their val sums Abar, Bbar, per train sample b
    sum_{x,y} (Abar A_b^T)[x, y] (Bbar B_b^T)[x, y], both Grams contracting over the L
    positions.  That is the fused ghost kernel with the i (= p) channel rows as its tokens, the
    positions as its features and the val block summed into one row; with bf16 operands the
    Gram entries and their products are rounded to bf16 as the reference's bf16 matmuls and
    multiply round them."""
    A_u = F.unfold(A.to(dtype), kernel_size=layer.kernel_size, dilation=layer.dilation,
                   padding=layer.padding, stride=layer.stride)
    B_r = B.to(dtype).reshape(B.size(0), B.size(1), -1)
    i, p = A_u.size(1), B_r.size(1)
    if i != p:
        raise RuntimeError(
            f"Conv2d ghost branch of the reference (reference_conv2d_ghost): its [{i}, {i}] "
            f"input Gram and [{p}, {p}] backprop Gram multiply elementwise only when "
            f"C_in*kh*kw ({i}) equals C_out ({p})")
    n_t = A_u.size(0) - n_val
    rows_a = torch.cat([A_u[:n_t], A_u[n_t:].sum(0, keepdim=True)])
    rows_b = torch.cat([B_r[:n_t], B_r[n_t:].sum(0, keepdim=True)])
    rounding = _native.ROUND_REF_BF16 if dtype == torch.bfloat16 else _native.ROUND_FP32
    dot, _ = _native.ops().linear_dot(rows_a, rows_b, 1, semantics=_native.SEM_PAIRWISE_SUM,
                                      algo=_native.ALGO_GHOST, rounding=rounding)
    return dot


def _compute_conv2d_dot_product(layer: nn.Conv2d, A: torch.Tensor, B: torch.Tensor,
                                val_batch_size: int) -> None:
    """Gradient dot-products of an nn.Conv2d (reference :513-560): unfold, then the presum
    dot of the per-sample weight gradients, dot_i = <sum_l b_il a_il^T, sum_l bbar_l abar_l^T>
    with abar, bbar the val sums, and the bias dot <sum_l b_il, sum_{j,l} b_jl>.

    Both of the reference's branches aim at this presum quantity; its materialised branch
    (:552-555) computes it, its ghost branch (:546-550) multiplies [d, d] by [p, p] blocks (it
    raises unless C_in*kh*kw == C_out).  The switch is still cached on the layer; with the
    option reference_conv2d_ghost a layer on the ghost branch gets that branch's quantity."""
    A = A.detach()
    B = B.detach()
    train_bs = A.size(0) - val_batch_size
    if train_bs <= 0:
        raise ValueError("No training samples to compute dot product")
    dt = torch.float32 if options["precision"] == "fp32" else torch.bfloat16
    A_rows, B_rows = _conv2d_rows(layer, A, B, dt)
    # The reference's switch on the unfolded shapes: T = L, 2 L^2 <= weight.numel().
    _should_use_ghost_computation(layer, A_rows.transpose(1, 2), B_rows.transpose(1, 2),
                                  conv=True)
    if options["reference_conv2d_ghost"] and layer.use_ghost_computation:
        layer.weight.grad_dot_prod = _conv2d_reference_ghost(layer, A, B, val_batch_size, dt)
    else:
        _linear_like_dot(layer, A_rows, B_rows, val_batch_size, False, dt)
    if layer.bias is not None:
        _bias_dot_and_grad(layer, B_rows, val_batch_size, dt)
    _reference_dtypes(layer, None if layer.use_ghost_computation else torch.bfloat16,
                      torch.bfloat16)


def _compute_conv2d_train_grad(layer: nn.Conv2d, A: torch.Tensor, B: torch.Tensor,
                               val_batch_size: int, scale: float = 1.0) -> torch.Tensor:
    """scale * sum over train rows and positions of b a^T / n_train, viewed as the weight
    (reference :563-592)."""
    n_t = A.size(0) - val_batch_size
    if n_t <= 0:
        return None
    dt = A.dtype if A.dtype in (torch.bfloat16, torch.float32) else torch.float32
    A_rows, B_rows = _conv2d_rows(layer, A[:n_t], B[:n_t], dt)
    grad = _scaled_mm(B_rows.reshape(-1, B_rows.shape[-1]).t(),
                      A_rows.reshape(-1, A_rows.shape[-1]), scale / n_t)
    return grad.view_as(layer.weight).to(layer.weight.dtype)


_supported_layers_dotprod = {
    nn.Linear: (_compute_linear_dot_product, _compute_linear_train_grad),
    nn.Embedding: (_compute_embedding_dot_product, _compute_embedding_train_grad),
    nn.LayerNorm: (_compute_layernorm_dot_product, _compute_layernorm_train_grad),
    nn.Conv2d: (_compute_conv2d_dot_product, _compute_conv2d_train_grad),
}
if _HFConv1D is not None:
    _supported_layers_dotprod[_HFConv1D] = (_compute_Conv1D_dot_product,
                                            _compute_Conv1D_train_grad)
