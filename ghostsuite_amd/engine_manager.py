"""GhostEngineManager: config-driven facade over the engines (mirrors
ghostEngines/engine_manager.py: method selection, train/val concatenation, save cadence,
evaluation detach/reattach and cleanup)."""
from __future__ import annotations

import os
from typing import Any, Dict

import torch
from torch import nn

from .graddotprod_engine import GradDotProdEngine
from .gradProjection.gradproj_engine import GradProjLoraEngine


class GhostEngineManager:
    """Owns one engine chosen by ``config.method`` in {'GradDotProd', 'GradProjLora',
    'Regular'} and exposes the training-loop calls."""

    def __init__(self, config, model: nn.Module, optimizer: torch.optim.Optimizer,
                 ddp_info: Dict[str, Any], val_data=None):
        self.config = config
        self.model = model
        self.optimizer = optimizer
        self.ddp_info = ddp_info
        self.engine = None
        if val_data is not None:
            self.X_val, self.Y_val = val_data
        else:
            self.X_val, self.Y_val = None, None
        self._initialize_engine()

    def _initialize_engine(self):
        if self.config.method == 'GradDotProd':
            self._initialize_graddotprod_engine()
        elif self.config.method == 'GradProjLora':
            self._initialize_gradproj_engine()
        elif self.config.method == 'Regular':
            print("[INFO] Regular training mode - no ghost engine required.")
        else:
            print(f"[WARNING] Unknown method '{self.config.method}' - no ghost engine initialized.")

    def _initialize_graddotprod_engine(self):
        print("[INFO] Initializing GradDotProdEngine ...")
        dot_prod_save_path = os.path.join(self.config.result_dir, "grad_dotprods")
        if self.ddp_info['master_process']:
            os.makedirs(dot_prod_save_path, exist_ok=True)
        self.engine = GradDotProdEngine(
            module=self.model,
            val_batch_size=self.config.val_batch_size,
            loss_reduction='mean',
            use_dummy_bias=True,
            dot_prod_save_path=dot_prod_save_path,
            **getattr(self.config, 'ghost_options', {}),
        )
        self.engine.attach(self.optimizer)
        if self.X_val is None or self.Y_val is None:
            raise ValueError("X_val and Y_val are required for GradDotProd method")
        self.engine.attach_and_store_valset(self.X_val, self.Y_val)
        print("[INFO] GradDotProdEngine initialized successfully.")

    def _initialize_gradproj_engine(self):
        print("[INFO] Initializing GradProjLoraEngine ...")
        proj_dir = os.path.join(self.config.result_dir, "projections")
        if self.ddp_info['master_process']:
            os.makedirs(proj_dir, exist_ok=True)
        self.engine = GradProjLoraEngine(
            module=self.model,
            proj_layers=getattr(self.config, 'proj_layers', 'mlp,attn'),
            proj_rank_total=getattr(self.config, 'proj_rank_total', 256),
            proj_rank_min=getattr(self.config, 'proj_rank_min', 8),
            proj_seed=getattr(self.config, 'proj_seed', 42),
            proj_dtype=getattr(self.config, 'proj_dtype', self.config.train_dtype),
            proj_dir=proj_dir,
            proj_save_interval=getattr(self.config, 'proj_save_interval',
                                       self.config.dot_prod_save_interval),
            include_embeddings=getattr(self.config, 'include_embeddings', False),
        )
        self.engine.attach()
        print("[INFO] GradProjLoraEngine initialized successfully.")

    def is_active(self) -> bool:
        return self.engine is not None

    def get_method(self) -> str:
        return self.config.method

    def attach_train_batch(self, X_train, Y_train, iter_num, batch_idx=None):
        if self.engine and hasattr(self.engine, 'attach_train_batch'):
            self.engine.attach_train_batch(X_train, Y_train, iter_num, batch_idx)

    def prepare_gradients(self):
        if self.engine and hasattr(self.engine, 'prepare_gradients'):
            self.engine.prepare_gradients()

    def aggregate_and_log(self):
        if self.engine and hasattr(self.engine, 'aggregate_and_log'):
            self.engine.aggregate_and_log()

    def clear_gradients(self):
        if self.engine and hasattr(self.engine, 'clear_gradients'):
            self.engine.clear_gradients()

    def should_save_metrics(self, iter_num: int) -> bool:
        if self.config.method == 'GradDotProd' and iter_num > 0:
            return iter_num % self.config.dot_prod_save_interval == 0
        elif self.config.method == 'GradProjLora' and iter_num > 0:
            save_interval = getattr(self.config, 'proj_save_interval',
                                    self.config.dot_prod_save_interval)
            return iter_num % save_interval == 0
        return False

    def save_metrics(self, iter_num: int):
        if self.config.method == 'GradDotProd' and self.engine:
            self.engine.save_dot_product_log(iter_num=iter_num)
        elif self.config.method == 'GradProjLora' and self.engine:
            if hasattr(self.engine, 'save_projections'):
                self.engine.save_projections(iter_num=iter_num)

    def get_validation_data(self):
        return self.X_val, self.Y_val

    def prepare_forward_input(self, X_train, Y_train):
        """Concatenates (train, val) for GradDotProd -- train rows first (reference :182-206)."""
        if self.config.method == 'GradDotProd' and self.X_val is not None:
            if isinstance(self.X_val, dict):
                X_cat = {k: torch.cat((X_train[k], self.X_val[k]), dim=0)
                         for k in ("input_ids", "pixel_values", "attention_mask")}
                return X_cat, torch.cat((Y_train, self.Y_val), dim=0)
            return torch.cat((X_train, self.X_val), dim=0), torch.cat((Y_train, self.Y_val), dim=0)
        return X_train, Y_train

    def detach_for_evaluation(self):
        if self.engine:
            if hasattr(self.engine, 'detach'):
                self.engine.detach()
            elif hasattr(self.engine, 'disable_hooks'):
                self.engine.disable_hooks()

    def reattach_after_evaluation(self):
        if self.engine:
            if hasattr(self.engine, 'attach'):
                if isinstance(self.engine, GradDotProdEngine):
                    self.engine.attach(self.optimizer)
                else:
                    self.engine.attach()
            elif hasattr(self.engine, 'enable_hooks'):
                self.engine.enable_hooks()

    def cleanup(self):
        """Saves what is left and detaches; errors are printed, not raised."""
        if not self.engine:
            return
        if (self.config.method == 'GradDotProd' and hasattr(self.engine, 'dot_product_log')
                and self.engine.dot_product_log):
            try:
                self.engine.save_dot_product_log(iter_num=-1)
            except Exception as e:
                print(f"Error saving remaining dot products during cleanup: {e}")
        elif self.config.method == 'GradProjLora':
            if hasattr(self.engine, 'cleanup'):
                try:
                    self.engine.cleanup()
                except Exception as e:
                    print(f"Error during GradProjLora cleanup: {e}")
        try:
            if hasattr(self.engine, 'detach'):
                self.engine.detach()
            elif hasattr(self.engine, 'disable_hooks'):
                self.engine.disable_hooks()
        except Exception as e:
            print(f"Error detaching ghost engine during cleanup: {e}")
