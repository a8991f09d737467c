"""Forward/backward hooks of GradProjLoRA (mirrors
ghostEngines/gradProjection/autograd_gradproj.py).

The backward hook hands the cached layer input A and the output grad B to the gfx950
Kronecker-projection kernel:
  nn.Linear:  _ghost_grad_proj[b] = B_batch * sum_t (P_o b_bt)(P_i a_bt)^T   [k_o, k_i]
  HF Conv1D:  _ghost_grad_proj[b] = B_batch * sum_t (P_i b_bt)(P_o a_bt)^T   [k_i, k_o]
(the reference's Conv1D role swap, :141-147).  Results are fp32.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _native, _overlap
from .._native import ops


def _flatten_tokens(x: torch.Tensor) -> torch.Tensor:
    """[B, ...] -> [B, T, D] (reference :11-37)."""
    if x.dim() <= 2:
        return x.unsqueeze(1)
    return x.reshape(x.shape[0], -1, x.shape[-1])


def _extract_batch_size(x: torch.Tensor) -> int:
    return 1 if x.dim() == 0 else x.shape[0]


class GradProjHooks:
    """Projection matrices of one layer and its forward/backward hooks."""

    def __init__(self, P_i: torch.Tensor, P_o: torch.Tensor, layer_name: str, layer_type: str):
        self.P_i = P_i
        self.P_o = P_o
        self.layer_name = layer_name
        self.layer_type = layer_type
        self._handle_forward = None
        self._handle_backward = None
        self._cast = {}

    def _proj(self, dtype: torch.dtype):
        """P_i, P_o in the operand dtype (converted once per dtype)."""
        if dtype not in self._cast:
            self._cast[dtype] = (self.P_i.to(dtype).contiguous(), self.P_o.to(dtype).contiguous())
        return self._cast[dtype]

    def forward_hook_store_inputs(self, module: nn.Module, inputs: Tuple[torch.Tensor, ...],
                                  output: torch.Tensor) -> None:
        module._ghost_A_raw = inputs[0].detach()

    def backward_hook_compute_proj(self, module: nn.Module,
                                   grad_input: Tuple[Optional[torch.Tensor], ...],
                                   grad_output: Tuple[torch.Tensor, ...]) -> None:
        A_raw = getattr(module, '_ghost_A_raw', None)
        if A_raw is None:
            raise RuntimeError(f'Missing cached activations for GradProjection in {self.layer_name}')
        B_out = grad_output[0]
        if B_out is None:
            module._ghost_grad_proj = None
            delattr(module, '_ghost_A_raw')
            return
        B_out = B_out.detach()
        # The projection kernels run on a side stream, overlapped with the rest of backward.
        with _overlap.on_side_stream(A_raw, B_out):
            if self.layer_type == 'Embedding':
                self._compute_embedding_proj(module, A_raw, B_out)
            else:
                self._compute_dense_proj(module, A_raw, B_out)
        delattr(module, '_ghost_A_raw')

    def _compute_dense_proj(self, module: nn.Module, A_raw: torch.Tensor,
                            B_out: torch.Tensor) -> None:
        """Projected per-sample gradients of a dense layer (reference :120-165)."""
        is_conv1d = module.__class__.__name__ == 'Conv1D'
        A = _flatten_tokens(A_raw)
        B = _flatten_tokens(B_out)
        batch_size = A.shape[0]
        dt = A.dtype if A.dtype in (torch.bfloat16, torch.float32) else torch.float32
        if A.dtype != dt:
            A = A.to(dt)
        if B.dtype != dt:
            B = B.to(dt)
        P_i, P_o = self._proj(dt)
        layout = _native.PROJ_KI_KO if is_conv1d else _native.PROJ_KO_KI
        module._ghost_grad_proj = ops().kron_proj(A, B, P_i, P_o, float(batch_size),
                                                  layout=layout, out_dtype=torch.float32)

    def _compute_embedding_proj(self, module: nn.Module, indices: torch.Tensor,
                                grad_output: torch.Tensor) -> None:
        """Projected per-sample gradients of an embedding (reference :167-222):
        sum_t (P_o g_t)(P_i[:, x_t])^T with no batch-size factor, as in the reference.  The
        gfx950 kernel gathers P_i's columns by token id on the device (the reference reads
        every id back to the host)."""
        bs = indices.shape[0]
        g = grad_output.reshape(bs, -1, grad_output.shape[-1])
        dt = g.dtype if g.dtype in (torch.bfloat16, torch.float32) else torch.float32
        if g.dtype != dt:
            g = g.to(dt)
        if ('embT', dt) not in self._cast:
            self._cast[('embT', dt)] = (self.P_i.t().to(dt).contiguous(),
                                        self.P_o.to(dt).contiguous())
        P_iT, P_o = self._cast[('embT', dt)]
        module._ghost_grad_proj = ops().kron_embed_proj(indices, g, P_iT, P_o, 1.0,
                                                        out_dtype=torch.float32)

    def attach(self, module: nn.Module) -> None:
        self._handle_forward = module.register_forward_hook(self.forward_hook_store_inputs)
        self._handle_backward = module.register_full_backward_hook(self.backward_hook_compute_proj)

    def detach(self) -> None:
        if self._handle_forward is not None:
            self._handle_forward.remove()
            self._handle_forward = None
        if self._handle_backward is not None:
            self._handle_backward.remove()
            self._handle_backward = None


def create_projection_hooks(module: nn.Module, layer_name: str, P_i: torch.Tensor,
                            P_o: torch.Tensor) -> GradProjHooks:
    """Hooks for one layer; Conv1d/Conv2d raise NotImplementedError as in the reference."""
    layer_type = module.__class__.__name__
    if layer_type == 'Conv1D':
        layer_type = 'Linear'
    elif isinstance(module, nn.Conv1d):
        raise NotImplementedError(
            f"Conv1d layers are not yet supported for gradient projection. Layer '{layer_name}' "
            "is a Conv1d layer. Proper im2col unfolding is required for correct gradient "
            "computation. Please exclude Conv1d layers from proj_layers pattern.")
    elif isinstance(module, nn.Conv2d):
        raise NotImplementedError(
            f"Conv2d layers are not yet supported for gradient projection. Layer '{layer_name}' "
            "is a Conv2d layer. Proper im2col unfolding is required for correct gradient "
            "computation. Please exclude Conv2d layers from proj_layers pattern or set "
            "include_conv2d=False.")
    elif isinstance(module, nn.Linear):
        layer_type = 'Linear'
    elif isinstance(module, nn.Embedding):
        layer_type = 'Embedding'
    else:
        raise ValueError(f"Unsupported layer type: {layer_type}")
    return GradProjHooks(P_i, P_o, layer_name, layer_type)
