"""GhostEngineManager: the one object a training loop talks to.

Keeps the reference's public surface (ghostEngines/engine_manager.py:18-253): the
constructor ``(config, model, optimizer, ddp_info, val_data)``, the engine chosen by
``config.method`` ('GradDotProd', 'GradProjLora' or 'Regular'), and the step protocol of
Examples/GradDotProd_LM/training_loop.py:99-166 -- attach_train_batch, prepare_forward_input
(train rows first, then the val rows), forward/backward, prepare_gradients, optimizer step,
aggregate_and_log, clear_gradients -- with should_save_metrics / save_metrics on the configured
interval, detach/reattach around evaluation and cleanup at the end.  ``config.ghost_options``
(a dict, optional) is passed to GradDotProdEngine as keyword options.
"""
from __future__ import annotations

import os
from typing import Any, Dict, Optional

import torch
from torch import nn

from .graddotprod_engine import GradDotProdEngine
from .gradProjection.gradproj_engine import GradProjLoraEngine

# Keys concatenated when the inputs are dicts (multimodal batches, reference :191-203).
_DICT_INPUT_KEYS = ("input_ids", "pixel_values", "attention_mask")


class GhostEngineManager:
    """Builds the engine ``config.method`` names and forwards the training-loop calls to it;
    every call is a no-op when there is no engine ('Regular' training)."""

    def __init__(self, config, model: nn.Module, optimizer: torch.optim.Optimizer,
                 ddp_info: Dict[str, Any], val_data=None):
        self.config = config
        self.model = model
        self.optimizer = optimizer
        self.ddp_info = ddp_info
        self.X_val, self.Y_val = val_data if val_data is not None else (None, None)
        self.engine: Optional[Any] = None
        builders = {"GradDotProd": self._build_graddotprod, "GradProjLora": self._build_gradproj}
        method = config.method
        if method in builders:
            builders[method]()
        elif method == "Regular":
            print("[INFO] Method 'Regular': plain training, no ghost engine.")
        else:
            print(f"[WARNING] Method '{method}' is not known; no ghost engine is used.")

    # ------------------------------------------------------------------ construction
    def _opt(self, name: str, default=None):
        return getattr(self.config, name, default)

    def _output_dir(self, leaf: str) -> str:
        path = os.path.join(self.config.result_dir, leaf)
        if self.ddp_info.get("master_process", True):
            os.makedirs(path, exist_ok=True)
        return path

    def _build_graddotprod(self):
        if self.X_val is None or self.Y_val is None:
            raise ValueError("X_val and Y_val are required for GradDotProd method")
        print("[INFO] Building GradDotProdEngine ...")
        self.engine = GradDotProdEngine(
            module=self.model, val_batch_size=self.config.val_batch_size,
            loss_reduction="mean", use_dummy_bias=True,
            dot_prod_save_path=self._output_dir("grad_dotprods"),
            **(self._opt("ghost_options") or {}))
        self.engine.attach(self.optimizer)
        self.engine.attach_and_store_valset(self.X_val, self.Y_val)

    def _build_gradproj(self):
        print("[INFO] Building GradProjLoraEngine ...")
        self.engine = GradProjLoraEngine(
            module=self.model,
            proj_layers=self._opt("proj_layers", "mlp,attn"),
            proj_rank_total=self._opt("proj_rank_total", 256),
            proj_rank_min=self._opt("proj_rank_min", 8),
            proj_seed=self._opt("proj_seed", 42),
            proj_dtype=self._opt("proj_dtype", self._opt("train_dtype")),
            proj_dir=self._output_dir("projections"),
            proj_save_interval=self._save_interval(),
            include_embeddings=self._opt("include_embeddings", False))
        self.engine.attach()

    # ------------------------------------------------------------------ forwarding
    def _call(self, name: str, *args, **kwargs):
        fn = getattr(self.engine, name, None) if self.engine is not None else None
        return fn(*args, **kwargs) if fn is not None else None

    def is_active(self) -> bool:
        return self.engine is not None

    def get_method(self) -> str:
        return self.config.method

    def get_validation_data(self):
        return self.X_val, self.Y_val

    def attach_train_batch(self, X_train, Y_train, iter_num, batch_idx=None):
        self._call("attach_train_batch", X_train, Y_train, iter_num, batch_idx)

    def prepare_gradients(self):
        self._call("prepare_gradients")

    def aggregate_and_log(self):
        self._call("aggregate_and_log")

    def clear_gradients(self):
        self._call("clear_gradients")

    # ------------------------------------------------------------------ saving
    def _save_interval(self) -> int:
        if self.config.method == "GradProjLora":
            return self._opt("proj_save_interval", self.config.dot_prod_save_interval)
        return self.config.dot_prod_save_interval

    def should_save_metrics(self, iter_num: int) -> bool:
        if iter_num <= 0 or self.config.method not in ("GradDotProd", "GradProjLora"):
            return False
        return iter_num % self._save_interval() == 0

    def save_metrics(self, iter_num: int):
        if self.engine is None:
            return
        if self.config.method == "GradDotProd":
            self.engine.save_dot_product_log(iter_num=iter_num)
        elif self.config.method == "GradProjLora":
            self._call("save_projections", iter_num=iter_num)

    # ------------------------------------------------------------------ the step's inputs
    def prepare_forward_input(self, X_train, Y_train):
        """GradDotProd runs one forward over the train rows followed by the val rows (the
        samplers split every layer's batch as [train, val]); other methods take the train
        batch as it is."""
        if self.config.method != "GradDotProd" or self.X_val is None:
            return X_train, Y_train
        Y = torch.cat((Y_train, self.Y_val), dim=0)
        if isinstance(self.X_val, dict):
            return {k: torch.cat((X_train[k], self.X_val[k]), dim=0) for k in _DICT_INPUT_KEYS}, Y
        return torch.cat((X_train, self.X_val), dim=0), Y

    # ------------------------------------------------------------------ evaluation / exit
    def _unhook(self):
        if hasattr(self.engine, "detach"):
            self.engine.detach()
        else:
            self._call("disable_hooks")

    def detach_for_evaluation(self):
        if self.engine is not None:
            self._unhook()

    def reattach_after_evaluation(self):
        if self.engine is None:
            return
        if isinstance(self.engine, GradDotProdEngine):
            self.engine.attach(self.optimizer)
        elif hasattr(self.engine, "attach"):
            self.engine.attach()
        else:
            self._call("enable_hooks")

    def cleanup(self):
        """Writes what the engine still holds, then removes its hooks; failures are printed
        so that the end of training is never interrupted."""
        if self.engine is None:
            return
        steps = []
        if self.config.method == "GradDotProd" and getattr(self.engine, "dot_product_log", None):
            steps.append(("saving the remaining dot products",
                          lambda: self.engine.save_dot_product_log(iter_num=-1)))
        elif self.config.method == "GradProjLora" and hasattr(self.engine, "cleanup"):
            steps.append(("GradProjLora cleanup", self.engine.cleanup))
        steps.append(("detaching the ghost engine", self._unhook))
        for what, fn in steps:
            try:
                fn()
            except Exception as e:  # noqa: BLE001 - reported, never raised at exit
                print(f"Error {what}: {e}")
