"""GradProjLoraEngine: per-sample projected gradients (mirrors
ghostEngines/gradProjection/gradproj_engine.py: layer matching, (k_i, k_o) choice, seeds
proj_seed + layer_idx for P_i and + 1000 for P_o in named_modules order, concatenation in
sorted layer-name order, cast to proj_dtype, proj_iter_{iter:06d}.pt + metadata.json)."""
from __future__ import annotations

import json
from collections import OrderedDict
from pathlib import Path
from typing import Dict, List, Optional, Tuple, Union

import torch
import torch.nn as nn

from .projection_utils import (choose_ki_ko, compute_projection_metadata,
                               get_projection_initializer)
from .. import _overlap, async_io
from .autograd_gradproj import create_projection_hooks
from .supported_layers_gradproj import (compute_total_projection_size, find_matching_layers,
                                        get_layer_dimensions, get_layer_slice_ranges,
                                        validate_layer_selection)


class GradProjLoraEngine:
    """Computes and stores per-sample projected gradients without changing training.

    ``proj_dims_override`` ({layer name: (k_i, k_o)} or a single (k_i, k_o) for every
    layer) replaces the choose_ki_ko rule when given.
    """

    def __init__(self, module: nn.Module, proj_layers: Union[str, List[str]],
                 proj_rank_total: int, proj_rank_min: int, proj_seed: int, proj_dtype: str,
                 proj_dir: str, proj_row_orthonormal: bool = False,
                 include_embeddings: bool = False, include_conv2d: bool = False,
                 proj_save_interval: int = 1, proj_dims_override=None, **kwargs):
        self.module = module
        self.proj_layers = proj_layers
        self.proj_rank_total = proj_rank_total
        self.proj_rank_min = proj_rank_min
        self.proj_seed = proj_seed
        self.proj_dir = Path(proj_dir)
        self.proj_save_interval = proj_save_interval
        dtype_map = {'float16': torch.float16, 'bfloat16': torch.bfloat16,
                     'float32': torch.float32}
        if proj_dtype not in dtype_map:
            raise ValueError(f"proj_dtype must be one of {list(dtype_map.keys())}, got {proj_dtype}")
        self.proj_dtype = dtype_map[proj_dtype]
        self.proj_method = 'orthonormal' if proj_row_orthonormal else 'gaussian'
        self.include_embeddings = include_embeddings
        self.include_conv2d = include_conv2d
        self.proj_dims_override = proj_dims_override
        self.matched_layers = OrderedDict()
        self.projection_matrices = {}
        self.projection_dims = {}
        self.hooks = {}
        self.slice_ranges = {}
        self.total_proj_dim = 0
        self.metadata = {}
        self.is_attached = False
        self.iteration = 0
        self.batch_count = 0
        self._initialize_projections()

    def _dims_for(self, name: str, n_i: int, n_o: int) -> Tuple[int, int]:
        ov = self.proj_dims_override
        if ov is None:
            return choose_ki_ko(n_i, n_o, self.proj_rank_total, self.proj_rank_min)
        if isinstance(ov, dict):
            if name in ov:
                return tuple(ov[name])
            return choose_ki_ko(n_i, n_o, self.proj_rank_total, self.proj_rank_min)
        return tuple(ov)

    def _initialize_projections(self):
        self.matched_layers = OrderedDict(find_matching_layers(
            self.module, self.proj_layers, self.include_embeddings, self.include_conv2d))
        validate_layer_selection(self.matched_layers, self.proj_layers)
        device = next(self.module.parameters()).device
        init_fn = get_projection_initializer(self.proj_method)
        torch.manual_seed(self.proj_seed)
        for layer_idx, (name, layer) in enumerate(self.matched_layers.items()):
            n_i, n_o = get_layer_dimensions(layer)
            k_i, k_o = self._dims_for(name, n_i, n_o)
            self.projection_dims[name] = (k_i, k_o)
            seed = self.proj_seed + layer_idx
            P_i = init_fn(k_i, n_i, dtype=torch.float32, device=device, seed=seed)
            P_o = init_fn(k_o, n_o, dtype=torch.float32, device=device, seed=seed + 1000)
            self.projection_matrices[name] = (P_i, P_o)
            print(f"  Projection dims: k_i={k_i}, k_o={k_o} (k_total={k_i * k_o})")
        self.slice_ranges = get_layer_slice_ranges(self.matched_layers, self.projection_dims)
        self.total_proj_dim = compute_total_projection_size(self.matched_layers,
                                                            self.projection_dims)
        print(f"Total projection dimension: {self.total_proj_dim}")
        self._prepare_metadata()

    def _prepare_metadata(self):
        self.metadata = {
            'engine': 'GradProjLora',
            'proj_seed': self.proj_seed,
            'proj_dtype': str(self.proj_dtype).split('.')[-1],
            'proj_method': self.proj_method,
            'proj_rank_total': self.proj_rank_total,
            'proj_rank_min': self.proj_rank_min,
            'total_proj_dim': self.total_proj_dim,
            'layers': [],
        }
        for name in sorted(self.matched_layers.keys()):
            k_i, k_o = self.projection_dims[name]
            start, end = self.slice_ranges[name]
            meta = compute_projection_metadata(name, self.matched_layers[name], k_i, k_o)
            meta['slice_start'] = start
            meta['slice_end'] = end
            self.metadata['layers'].append(meta)

    def attach(self):
        if self.is_attached:
            return
        for name, layer in self.matched_layers.items():
            P_i, P_o = self.projection_matrices[name]
            hooks = create_projection_hooks(layer, name, P_i, P_o)
            hooks.attach(layer)
            self.hooks[name] = hooks
        self.is_attached = True
        print(f"Attached projection hooks to {len(self.matched_layers)} layers")

    def detach(self):
        if not self.is_attached:
            return
        for name, hooks in self.hooks.items():
            hooks.detach()
            layer = self.matched_layers[name]
            for attr in ('_ghost_A_raw', '_ghost_grad_proj'):
                if hasattr(layer, attr):
                    delattr(layer, attr)
        self.hooks.clear()
        self.is_attached = False
        async_io.writer.flush()   # projection files submitted so far are on disk
        print(f"Detached projection hooks from {len(self.matched_layers)} layers")

    def collect_batch(self, batch_indices: Optional[List[int]] = None) -> torch.Tensor:
        """[B, total_proj_dim] in proj_dtype, layers in sorted-name order; saved every
        proj_save_interval calls."""
        if not self.is_attached:
            raise RuntimeError("Engine is not attached. Call attach() first.")
        _overlap.join()   # the projection kernels run on the side stream
        parts, batch_size = [], None
        for name in sorted(self.matched_layers.keys()):
            grad_proj = getattr(self.matched_layers[name], '_ghost_grad_proj', None)
            if grad_proj is None:
                raise RuntimeError(f"No projected gradient found for layer {name}")
            B, k_o, k_i = grad_proj.shape
            if batch_size is None:
                batch_size = B
            elif B != batch_size:
                raise RuntimeError(f"Batch size mismatch: expected {batch_size}, got {B} for {name}")
            parts.append(grad_proj.reshape(B, k_i * k_o))
        full = torch.cat(parts, dim=1).to(self.proj_dtype)
        if self.iteration % self.proj_save_interval == 0:
            self._save_projection(full, batch_indices)
        self.iteration += 1
        self.batch_count += batch_size
        return full

    def _save_projection(self, projection: torch.Tensor, batch_indices: Optional[List[int]] = None):
        self.proj_dir.mkdir(parents=True, exist_ok=True)
        metadata_path = self.proj_dir / 'metadata.json'
        if not metadata_path.exists():
            with open(metadata_path, 'w') as f:
                json.dump(self.metadata, f, indent=2)
            print(f"Saved metadata to {metadata_path}")
        # The host copy and the file write leave the step's critical path: pinned copy on a
        # copy stream, torch.save on the writer thread once the copy is done.
        events = []
        save_dict = {'proj': async_io.tree_to_host_async(projection, events),
                     'iter': self.iteration, 'batch_size': projection.shape[0]}
        if batch_indices is not None:
            save_dict['batch_idx'] = batch_indices
        save_path = self.proj_dir / f'proj_iter_{self.iteration:06d}.pt'
        async_io.writer.submit(save_dict, save_path, events)
        print(f"Saved projection [{projection.shape}] to {save_path}")

    def get_projection_metadata(self) -> dict:
        return self.metadata.copy()

    # --- engine-manager compatibility (reference :303-430; the later aggregate_and_log wins)
    def attach_train_batch(self, X_train, Y_train, iter_num, batch_idx=None):
        self.current_iter_num = iter_num
        self.current_batch_idx = batch_idx

    def prepare_gradients(self):
        pass

    def aggregate_and_log(self):
        """Calls collect_batch() (with the attached batch indices when present)."""
        if getattr(self, 'current_batch_idx', None) is not None:
            self.collect_batch(batch_indices=self.current_batch_idx)
        else:
            self.collect_batch()

    def clear_gradients(self):
        for layer in self.matched_layers.values():
            for attr in ('_ghost_A_raw', '_ghost_grad_proj'):
                if hasattr(layer, attr):
                    delattr(layer, attr)

    def attach_with_optimizer(self, optimizer):
        self.attach()

    def detach_for_evaluation(self):
        self.detach()

    def reattach_after_evaluation(self):
        if not self.is_attached:
            self.attach()

    def cleanup(self):
        self.detach()
        self.projection_matrices.clear()

    def save_projections(self, iter_num: int):
        """Projections are saved by ``collect_batch``; this waits until they are on disk."""
        async_io.writer.flush()

    def __repr__(self):
        return (f"GradProjLoraEngine(layers={len(self.matched_layers)}, "
                f"total_dim={self.total_proj_dim}, attached={self.is_attached})")


# The README's spelling.
GradProjLoRAEngine = GradProjLoraEngine


def create_gradproj_engine(model: nn.Module, config: dict) -> GradProjLoraEngine:
    for param in ['proj_layers', 'proj_rank_total', 'proj_rank_min', 'proj_seed', 'proj_dtype',
                  'proj_dir']:
        if param not in config:
            raise ValueError(f"Missing required parameter: {param}")
    return GradProjLoraEngine(model, **config)
