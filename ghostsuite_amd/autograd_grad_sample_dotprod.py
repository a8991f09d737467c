"""Autograd hooks of the GradDotProd engine.

Mirrors ghostEngines/autograd_grad_sample_dotprod.py: a forward hook caches each supported
layer's input; a full backward hook computes the layer's gradient dot products, then its
train gradients, then frees the caches.  Differences are internal only:
  - the N-scaling of the backprops for loss_reduction='mean' (:132-134) is carried as a
    scalar (``layer.backprops_scale``) instead of a scaled copy of the backprops;
  - bias and LayerNorm train gradients come out of the same kernel pass as their dots;
  - a forward sequence stamp lets a tied Linear skip the dot that the Embedding sharing its
    weight overwrites later in the same backward.
"""
from __future__ import annotations

import contextlib
import itertools
from typing import Tuple

import torch
import torch.nn as nn

from . import _overlap
from .supported_layers_grad_samplers_dotprod import (
    APPLIED,
    _supported_layers_dotprod,
    _create_or_accumulate_train_grad,
    options,
)

_step_counter = itertools.count()
_fwd_counter = itertools.count()
_current_step = [0]


def requires_grad(module: nn.Module) -> bool:
    """True if any parameter of the module was trainable before the engine took over."""
    return any(p.initially_requires_grad for p in module.parameters())


def add_hooks(model: nn.Module, val_batch_size: int, loss_reduction: str = 'mean'):
    """Registers the forward/backward hooks on every supported layer with a trainable
    parameter (reference :23-81).  Raises ValueError when hooks are already present."""
    if hasattr(model, "autograd_grad_sample_hooks"):
        raise ValueError("Trying to add hooks twice to the same model")

    handles = []
    embeddings_by_weight = {}
    linears = []
    for name, layer in model.named_modules():
        if type(layer) in _supported_layers_dotprod and requires_grad(layer):
            handles.append(layer.register_forward_hook(_capture_activations))
            layer.name = name

            def backward_hook(this_layer, grad_input, grad_output):
                _prepare_sample_grad_or_dotprod(this_layer, grad_output, val_batch_size,
                                                loss_reduction)
                _apply_train_grad(this_layer, val_batch_size)
                return None

            handles.append(layer.register_full_backward_hook(backward_hook))
            if isinstance(layer, nn.Embedding):
                embeddings_by_weight[id(layer.weight)] = layer
            elif isinstance(layer, nn.Linear):
                linears.append(layer)
        else:
            is_atomic_layer = not list(layer.children())
            if is_atomic_layer and requires_grad(layer):
                print(f"WARNING: Skipping atomic layer '{name}' of type {type(layer)} "
                      "because it is not supported.")

    for lin in linears:
        emb = embeddings_by_weight.get(id(lin.weight))
        if emb is not None:
            # A plain attribute, not a registered submodule: the model's modules and
            # state_dict keys stay as they were.
            lin.__dict__["_gs_tied_embedding"] = emb
    handles.append(model.register_forward_pre_hook(_new_step))
    model.__dict__.setdefault("autograd_grad_sample_hooks", []).extend(handles)


def remove_hooks(model: nn.Module):
    """Removes hooks added by ``add_hooks()``."""
    if hasattr(model, "autograd_grad_sample_hooks"):
        for handle in model.autograd_grad_sample_hooks:
            handle.remove()
        del model.autograd_grad_sample_hooks
    for layer in model.modules():
        layer.__dict__.pop("_gs_tied_embedding", None)


def _new_step(module, inputs):
    _current_step[0] = next(_step_counter)


def _capture_activations(layer: nn.Module, inputs: Tuple, outputs: Tuple):
    """Forward hook: caches the (detached) layer input (reference :92-94)."""
    layer.activations = inputs[0].detach()
    layer._gs_fwd_seq = (_current_step[0], next(_fwd_counter))


def _prepare_sample_grad_or_dotprod(layer: nn.Module, grad_output: Tuple[torch.Tensor],
                                    val_batch_size: int, loss_reduction: str = 'mean'):
    """Backward-hook stage 1: the layer's dot products (reference :97-137)."""
    backprops = grad_output[0].detach()
    if not hasattr(layer, 'activations'):
        layer.activations = None
    compute_layer_dotprod, _ = _supported_layers_dotprod.get(type(layer))

    scale = float(backprops.shape[0]) if loss_reduction == 'mean' else 1.0
    n_train = backprops.shape[0] - val_batch_size
    if n_train > 0:
        # Train-gradient scales for the fused bias / LayerNorm passes.  The bias path always
        # divides by n_train (_apply_train_grad is called without loss_reduction, :67).
        layer._gs_bias_grad_scale = scale / n_train
        layer._gs_ln_grad_scale = scale / n_train

    acts = layer.activations
    # The dot kernels run on a side stream, overlapped with the rest of backward.
    side = _overlap.on_side_stream(acts, backprops) if options["overlap"] else \
        contextlib.nullcontext()
    with side:
        if acts is not None and acts.dtype != backprops.dtype and acts.is_floating_point():
            common = torch.promote_types(acts.dtype, backprops.dtype)
            compute_layer_dotprod(layer, acts.to(common), backprops.to(common),
                                  val_batch_size=val_batch_size)
        elif acts is not None and acts.dtype != backprops.dtype and \
                options["reference_id_promotion"]:
            # The reference promotes integer token ids to the backprops' dtype too (:116-123),
            # which rounds ids >= 256 in a bf16 model before its sampler casts them back.
            common = torch.promote_types(acts.dtype, backprops.dtype)
            compute_layer_dotprod(layer, acts.to(common).long(), backprops,
                                  val_batch_size=val_batch_size)
        else:
            compute_layer_dotprod(layer, acts, backprops, val_batch_size=val_batch_size)

    layer.backprops = backprops
    layer.backprops_scale = scale


def _apply_train_grad(layer: nn.Module, val_batch_size: int, loss_reduction: str = 'mean'):
    """Backward-hook stage 2: train gradients into ``param.train_grad`` (reference :140-196)."""
    _, compute_layer_train_grad = _supported_layers_dotprod.get(type(layer), (None, None))
    if not compute_layer_train_grad:
        raise ValueError(
            f"Layer {layer.__class__.__name__} is not supported for training gradient "
            "computation. Ensure it is included in the _supported_layers_dotprod dictionary.")
    scale = getattr(layer, "backprops_scale", 1.0)
    # The train-gradient kernels join the layer's dot kernels on the side stream: both read
    # only this layer's activations and backprops, and the end-of-backward join orders
    # param.train_grad before the optimizer reads it.  When the dot stage already formed
    # every train gradient, nothing is enqueued here but an add_ into an existing train_grad
    # (after a join), so the side stream is left alone.
    side = _overlap.on_side_stream(layer.__dict__.get("activations"),
                                   layer.__dict__.get("backprops")) \
        if options["overlap"] and not _train_grads_parked(layer) else contextlib.nullcontext()
    try:
        with side:
            _apply_train_grad_body(layer, compute_layer_train_grad, val_batch_size, scale,
                                   loss_reduction)
    finally:
        for attr in ('activations', 'backprops', 'backprops_scale', '_gs_bias_train_grad',
                     '_gs_weight_train_grad', '_gs_ln_train_grads', '_gs_bias_grad_scale',
                     '_gs_ln_grad_scale'):
            layer.__dict__.pop(attr, None)


def _train_grads_parked(layer: nn.Module) -> bool:
    """True when the dot stage parked every train gradient this layer applies."""
    d = layer.__dict__
    if isinstance(layer, nn.LayerNorm):
        return "_gs_ln_train_grads" in d
    w = getattr(layer, "weight", None)
    if w is None or not getattr(w, "initially_requires_grad", False) or \
            "_gs_weight_train_grad" not in d:
        return False
    b = getattr(layer, "bias", None)
    return b is None or not getattr(b, "initially_requires_grad", False) or \
        "_gs_bias_train_grad" in d


def _apply_train_grad_body(layer: nn.Module, compute_layer_train_grad, val_batch_size: int,
                           scale: float, loss_reduction: str):
    """The train gradients of one layer (weight, then bias) into ``param.train_grad``."""
    if isinstance(layer, nn.LayerNorm):
        compute_layer_train_grad(layer, layer.activations, layer.backprops, val_batch_size,
                                 scale=scale)
    else:
        if hasattr(layer, 'weight') and layer.weight.initially_requires_grad:
            grad_weight = compute_layer_train_grad(layer, layer.activations, layer.backprops,
                                                   val_batch_size, scale=scale)
            if grad_weight is APPLIED:
                pass   # the sampler added into param.train_grad itself
            elif grad_weight is not None:
                _create_or_accumulate_train_grad(layer.weight, grad_weight)
            else:
                raise ValueError(
                    f"Layer {layer.__class__.__name__} returned None for weight gradient. "
                    "Ensure the compute_layer_train_grad function is implemented correctly.")
        if hasattr(layer, 'bias') and layer.bias is not None and \
                layer.bias.initially_requires_grad:
            grad_bias = layer.__dict__.pop("_gs_bias_train_grad", None)
            if grad_bias is None:
                grad_bias = _compute_train_grad_bias(layer.backprops, val_batch_size,
                                                     loss_reduction=loss_reduction)
                if scale != 1.0:
                    grad_bias = grad_bias * scale
            _create_or_accumulate_train_grad(layer.bias, grad_bias)


def _compute_train_grad_bias(B: torch.Tensor, val_batch_size: int,
                             loss_reduction: str = 'mean') -> torch.Tensor:
    """Sum (or mean over train rows, for 'mean') of the train rows of B, per feature
    (reference :199-222)."""
    train_batch_size = B.size(0) - val_batch_size
    if train_batch_size <= 0:
        raise ValueError("No training samples to compute gradients, check batch sizes.")
    B_train = B[:train_batch_size]
    summed = B_train.sum(dim=list(range(B_train.dim() - 1)))
    if loss_reduction == 'mean':
        summed /= train_batch_size
    return summed
