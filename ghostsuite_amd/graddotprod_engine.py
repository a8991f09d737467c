"""GradDotProdEngine: in-run gradient dot products between a val batch and each train row.

Public behaviour mirrors ghostEngines/graddotprod_engine.py (constructor, attach/detach,
prepare_gradients, clear_gradients, aggregate_and_log, save_dot_product_log,
attach_and_store_valset, attach_train_batch, the dot_product_log record format).  Extra
keyword arguments set the sampler options of
``supported_layers_grad_samplers_dotprod.options`` (precision, linear_algo, rounding,
store_pairs, skip_overwritten_tied_dots, record_algorithms, overlap,
reference_id_promotion, reference_conv2d_ghost, dot_dtypes).  Options belong to the engine:
each starts from the defaults, and the engine whose model runs its forward installs its own
into the shared dict the samplers read, keeping direct changes made to that dict while it
was the one installed.
"""
from __future__ import annotations

import os
import warnings
import weakref
from typing import Optional

import torch
from torch import nn

from . import _overlap
from . import async_io
from . import autograd_grad_sample_dotprod
from . import transformers_support
from . import supported_layers_grad_samplers_dotprod as _samplers


class GradDotProdEngine:
    """Computes per-train-row dot products with the val gradient during backward and
    supplies the train-row gradient to the optimizer."""

    def __init__(self, module: nn.Module, val_batch_size: int, loss_reduction: str = 'mean',
                 use_dummy_bias: bool = False, dot_prod_save_path: Optional[str] = None,
                 **sampler_options):
        super().__init__()
        unknown = set(sampler_options) - set(_samplers.options)
        if unknown:
            raise TypeError(f"unknown GradDotProdEngine options: {sorted(unknown)}")
        # Options apply per engine: nothing an earlier engine set carries over.
        self._options = dict(_samplers.DEFAULT_OPTIONS)
        self._options.update(sampler_options)
        self._options_hook = None
        self._activate_options()

        self.module = module
        self.val_batch_size = val_batch_size
        self.loss_reduction = loss_reduction
        self.dot_prod_save_path = dot_prod_save_path
        self.named_params = list((n, p) for (n, p) in module.named_parameters() if p.requires_grad)
        self._grad_creation_locked = False
        # Records are appended with their device->host copies in flight; reads wait for them.
        self.dot_product_log = async_io.PendingLog()
        self.batch_idx_lst = []

        # Dummy-bias trick (reference :64-73): remember trainability, then let autograd skip
        # every weight-grad GEMM when enabled; the hooks supply the train gradients.
        for _, param in module.named_parameters():
            param.initially_requires_grad = bool(param.requires_grad)
            param.requires_grad = not use_dummy_bias

        transformers_support.forward_swapper(module=module)

    @property
    def options(self) -> dict:
        """This engine's sampler options: the shared dict while they are installed."""
        return _samplers.options if _options_owner() is self else self._options

    def _activate_options(self, *_):
        """Installs this engine's options into the shared dict the samplers read (a forward
        pre-hook of the model once attached).  The engine installed before keeps the values
        the shared dict holds now, direct changes included."""
        global _options_owner
        prev = _options_owner()
        if prev is self:
            return
        if prev is not None:
            prev._options = dict(_samplers.options)
        _samplers.options.clear()
        _samplers.options.update(self._options)
        _options_owner = weakref.ref(self)

    def _lock_grad_creation(self):
        self._grad_creation_locked = True

    def _unlock_grad_creation(self):
        self._grad_creation_locked = False

    def attach(self, optimizer: torch.optim.Optimizer):
        """Registers the hooks and keeps a back-reference on the optimizer."""
        self.optimizer = optimizer
        autograd_grad_sample_dotprod.add_hooks(model=self.module,
                                               val_batch_size=self.val_batch_size,
                                               loss_reduction=self.loss_reduction)
        self._activate_options()
        self._options_hook = self.module.register_forward_pre_hook(self._activate_options)
        optimizer.grad_dot_prod_engine = self

    def detach(self):
        """Removes the hooks and the engine's per-parameter attributes."""
        optimizer = self.optimizer
        if hasattr(optimizer, "grad_dot_prod_engine"):
            del optimizer.grad_dot_prod_engine
        autograd_grad_sample_dotprod.remove_hooks(self.module)
        if self._options_hook is not None:
            self._options_hook.remove()
            self._options_hook = None
        self.module.zero_grad()
        for param in self.module.parameters():
            for attr in ('train_grad', 'grad_dot_prod', 'grad_dot_prod_pair', 'activations',
                         'backprops'):
                if hasattr(param, attr):
                    delattr(param, attr)

    def _prepare_and_apply_train_grad(self):
        """Moves ``param.train_grad`` into ``param.grad`` (reference :131-163)."""
        if self._grad_creation_locked:
            return
        _overlap.join()   # fused bias / LayerNorm train grads come from the side stream
        for name, param in self.module.named_parameters():
            if not param.initially_requires_grad:
                continue
            if "dummy_bias" in name:
                continue
            if hasattr(param, 'train_grad'):
                if param.train_grad is None:
                    raise ValueError(
                        f"Parameter {name} requires grad has no accumulated training gradient. ")
                param.grad = param.train_grad
            else:
                raise ValueError(
                    f"Parameter {name} requires grad but does not have 'train_grad' attribute. ")
        self._lock_grad_creation()

    def _clear_train_grad(self):
        for param in self.module.parameters():
            if hasattr(param, 'train_grad'):
                del param.train_grad
        self._unlock_grad_creation()

    def prepare_gradients(self):
        """Move accumulated training gradients to ``.grad`` for the optimizer."""
        self._prepare_and_apply_train_grad()

    def clear_gradients(self):
        """Remove stored training gradients after the optimizer step."""
        self._clear_train_grad()

    def aggregate_and_log(self):
        """Aggregate per-layer dot products and append them to the log."""
        self._aggregate_and_log_dot_products()

    def _aggregate_and_log_dot_products(self):
        """Sums ``grad_dot_prod`` over parameters in ``named_parameters`` order -- the first
        tensor accumulates the rest in place -- and logs a CPU copy (reference :192-230)."""
        _overlap.join()
        dots = []
        for _, param in self.module.named_parameters():
            if hasattr(param, 'grad_dot_prod') and param.initially_requires_grad:
                if param.grad_dot_prod.numel() > 0:
                    dots.append(param.grad_dot_prod)
                delattr(param, 'grad_dot_prod')
            if hasattr(param, 'grad_dot_prod_pair'):
                delattr(param, 'grad_dot_prod_pair')
        total = _sum_into_first(dots) if dots else None
        if total is not None:
            # Same record as the reference, but the host copies are asynchronous (pinned
            # memory, copy stream): the step does not wait for the GPU here.
            events = []
            self.dot_product_log.append_pending({
                'dot_product': async_io.tree_to_host_async(total, events),
                'X_train': async_io.tree_to_host_async(self.X_train, events),
                'Y_train': async_io.tree_to_host_async(self.Y_train, events),
                'iter_num': self.iter_num,
                'batch_idx': self.batch_idx,
            }, events)
        else:
            warnings.warn("No gradient dot products computed for this iteration.")

    def save_dot_product_log(self, iter_num: int):
        """Writes ``dot_prod_log_iter_{iter_num}.pt`` (a list of the per-step records)."""
        if not self.dot_product_log:
            raise ValueError("No gradient dot products found to save for this iteration.")
        print(f"[INFO] Saving dot product log at iteration {iter_num} ...")
        file_path = os.path.join(self.dot_prod_save_path, f"dot_prod_log_iter_{iter_num}.pt")
        torch.save(self.dot_product_log.plain(), file_path)   # a plain list, as the reference
        self.dot_product_log.clear()

    def attach_and_store_valset(self, X_val, Y_val):
        """Writes ``valset.pt`` = {'X_val', 'Y_val'} on the CPU."""
        valset_path = os.path.join(self.dot_prod_save_path, "valset.pt")
        torch.save({'X_val': to_device(X_val, 'cpu'), 'Y_val': to_device(Y_val, 'cpu')},
                   valset_path)
        print(f"[INFO] Saved validation set to {valset_path}")

    def attach_train_batch(self, X_train, Y_train, iter_num, batch_idx=None):
        """Records the current train batch for the log."""
        self.X_train = X_train
        self.Y_train = Y_train
        self.iter_num = iter_num
        self.batch_idx = batch_idx


def _sum_into_first(dots):
    """dots[0] += dots[1], += dots[2], ... in order, in place (reference :204-211).  GPU tensors
    take one ordered-sum launch: the same fp32 adds in the same order, each rounded to the
    first tensor's dtype, as the in-place adds round them (one kernel instead of one per
    parameter; a bf16 dot added into an fp32 total would otherwise take torch's mixed-dtype
    add, ~38 us each on this GPU).  Other tensors are added one by one."""
    from . import _native
    total = dots[0]
    if len(dots) > 1 and total.is_cuda and all(
            d.device == total.device and d.is_contiguous() and d.numel() == total.numel() and
            d.dtype in (torch.float32, torch.bfloat16) for d in dots):
        return _native.ops().ordered_sum_(dots)
    for d in dots[1:]:
        total += d
    return total


def _no_owner():
    return None


# The engine whose options the shared dict holds (a weak reference).
_options_owner = _no_owner


def to_device(data, device):
    """Move a tensor, or each tensor of a dict, to ``device``."""
    if isinstance(data, dict):
        return {k: v.to(device) if hasattr(v, 'to') else v for k, v in data.items()}
    elif hasattr(data, 'to'):
        return data.to(device)
    raise TypeError(f"Unsupported data type for moving to GPU: {type(data)}. "
                    "Expected tensor or dict of tensors.")
