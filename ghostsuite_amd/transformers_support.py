"""Model-compatibility pieces the engines rely on.

Two behaviours of ghostEngines/transformers_support.py are kept:
  - ``_add_dummy_bias`` (:17-37): a zero, trainable ``dummy_bias`` added to an embedding's
    output keeps the autograd graph alive when every weight has requires_grad=False;
  - per-sample position ids (:228-231): a position embedding must see [B, T] ids so that
    its backward hook gets per-sample gradients.
``forward_swapper`` applies them to models that declare their embeddings through
``ghost_embeddings`` (the workload models of this package).  Hugging Face forward swaps
are not part of this build (they target transformers 4.x internals).
"""
from __future__ import annotations

import types
import warnings

import torch
from torch import nn


def _add_dummy_bias(embedding: nn.Embedding):
    """Adds a zero ``dummy_bias`` parameter to the embedding output and freezes the weight."""
    if hasattr(embedding, "dummy_bias"):
        return
    embedding.register_parameter(
        "dummy_bias", nn.Parameter(torch.zeros(1, device=embedding.weight.device)))
    old_forward = embedding.forward

    def new_forward(self, input, *args, **kwargs):
        output = old_forward(input, *args, **kwargs)
        bias = self.dummy_bias.to(dtype=output.dtype, device=output.device)
        return output + bias * 0

    embedding.forward = types.MethodType(new_forward, embedding)
    embedding.weight.requires_grad = False
    embedding.dummy_bias.initially_requires_grad = True


def forward_swapper(module: nn.Module):
    """Adds dummy biases to the embeddings a model lists in ``ghost_embeddings``; other
    plain nn.Modules are left untouched (reference :41-69 does nothing for them either)."""
    names = getattr(module, "ghost_embeddings", None)
    if names:
        for name in names:
            _add_dummy_bias(module.get_submodule(name))
        return
    try:
        import transformers
        if isinstance(module, transformers.PreTrainedModel):
            warnings.warn(f"{module.__class__.__name__}: Hugging Face forward swapping is not "
                          "provided; position embeddings may see broadcast ids.")
    except Exception:
        pass
