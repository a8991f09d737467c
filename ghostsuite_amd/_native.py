"""ctypes binding of libghost_hip.so (include/ghost_hip.h) and torch-tensor wrappers.

Every wrapper takes device tensors, checks shapes on the host, sizes and allocates the
workspace from torch's caching allocator, and launches on torch's current stream; no call
synchronises.  There is no CPU path: a tensor that is not on a ROCm device, or a missing
library, raises.

Host-logic tests swap the kernel layer for a checker through ``_install_backend`` (the
samplers call ``ops()``); product code never does.
"""
from __future__ import annotations

import ctypes
import threading
from typing import Optional, Tuple

import torch

from . import build as _build

# gs_dtype / gs_semantics / gs_algo / gs_rounding / gs_proj_layout (include/ghost_hip.h)
DTYPE_BF16, DTYPE_F32, DTYPE_F16 = 0, 1, 2
SEM_PAIRWISE_SUM, SEM_PRESUM = 0, 1
ALGO_AUTO, ALGO_GHOST, ALGO_VALGRAD = 0, 1, 2
ROUND_FP32, ROUND_REF_BF16 = 0, 1
PROJ_KO_KI, PROJ_KI_KO = 0, 1
ERR_UNSUPPORTED = -5  # gs_status GS_ERR_UNSUPPORTED: a valid request outside the kernels' limits
ABI_VERSION = 2

_TORCH_TO_GS = {torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32, torch.float16: DTYPE_F16}
ALGO_NAMES = {ALGO_AUTO: "auto", ALGO_GHOST: "ghost", ALGO_VALGRAD: "valgrad"}


class GhostHipError(RuntimeError):
    """A libghost_hip.so entry point returned an error status."""


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

_I64 = ctypes.c_int64
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "gs_abi_version": (_I, []),
    "gs_last_error": (ctypes.c_char_p, []),
    "gs_linear_dot_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64, _I, _I, _I]),
    "gs_linear_dot_algo": (_I, [_I, _I64, _I64, _I64, _I64, _I64, _I, _I, _I]),
    "gs_linear_dot": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I,
                           _P, _P, _P, _SZ, _P]),
    "gs_linear_dot_noalloc_bytes": (_SZ, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I, _I,
                                         _I]),
    "gs_linear_dot_noalloc": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I,
                                   _I, _P, _P, _P]),
    "gs_bias_dot_workspace": (_SZ, [_I64, _I64, _I64]),
    "gs_bias_dot": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _P, _I, _F, _P, _SZ, _P]),
    "gs_embedding_dot_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "gs_embedding_dot": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _SZ,
                              _P]),
    "gs_embedding_train_grad_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "gs_embedding_train_grad": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P,
                                     _I, _I, _P, _SZ, _P]),
    "gs_layernorm_dot_workspace": (_SZ, [_I64, _I64, _I64]),
    "gs_layernorm_dot": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P,
                              _I, _F, _P, _SZ, _P]),
    "gs_kron_proj_workspace": (_SZ, [_I64, _I64, _I64, _I64]),
    "gs_kron_proj": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _I, _I64, _I64, _I, _F,
                          _P, _I, _P, _SZ, _P]),
    "gs_kron_embed_proj": (_I, [_P, _P, _I, _I64, _I64, _I64, _P, _P, _I, _I64, _I64, _I64, _F,
                                _P, _I, _P, _SZ, _P]),
    "gs_linear_rowdot_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64]),
    "gs_linear_val_gradient_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64, _I]),
    "gs_linear_val_gradient": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P,
                                    _P, _SZ, _P]),
    "gs_linear_dot_train_grad_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64, _I, _I]),
    "gs_linear_dot_train_grad": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P,
                                      _P, _I, _F, _P, _P, _I, _F, _P, _SZ, _P]),
    "gs_conv1d_dot_train_grad_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64, _I, _I]),
    "gs_conv1d_dot_train_grad": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P,
                                      _P, _I, _F, _P, _P, _I, _F, _P, _SZ, _P]),
    "gs_linear_train_grad_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64]),
    "gs_linear_train_grad": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I,
                                  _I, _P, _SZ, _P]),
    "gs_linear_rowdot_bias_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64]),
    "gs_linear_rowdot_bias": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P,
                                   _P, _I, _F, _P, _SZ, _P]),
    "gs_linear_rowdot": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _SZ,
                              _P]),
    "gs_linear_bias_dot_workspace": (_SZ, [_I, _I64, _I64, _I64, _I64, _I64, _I]),
    "gs_linear_bias_dot": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _P, _P,
                                _I, _F, _P, _SZ, _P]),
    "gs_ordered_sum": (_I, [_P, _P, _I, _I64, _P, _I, _P]),
}


def load_library() -> ctypes.CDLL:
    """Loads libghost_hip.so (built in-tree by ghostsuite_amd.build) once per process."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = _build.library_path()
        if not path.exists():
            raise GhostHipError(
                f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python ghostsuite_amd/build.py` first")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.gs_abi_version()
        if ver != ABI_VERSION:
            raise GhostHipError(f"libghost_hip ABI {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def exported_symbols() -> list:
    return list(_SIGNATURES)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().gs_last_error().decode(errors="replace")
        raise GhostHipError(f"{what} failed ({rc}): {msg}")


def _gs_dtype(t: torch.Tensor) -> int:
    try:
        return _TORCH_TO_GS[t.dtype]
    except KeyError:
        raise GhostHipError(f"unsupported dtype {t.dtype}") from None


def _require_device(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise GhostHipError(
                "ghostsuite_amd kernels need tensors on a ROCm GPU device; got a tensor on "
                f"{t.device} (there is no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise GhostHipError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def _tokens(x: torch.Tensor, n: int, feat: int) -> int:
    if x.dim() < 2 or x.shape[0] != n:
        raise GhostHipError(f"expected a [N, ..., F] tensor with N={n}, got {tuple(x.shape)}")
    return x.numel() // (n * feat) if n * feat > 0 else 0


class HipOps:
    """The kernel layer the samplers call: one C-ABI call per op, async on the current stream."""

    name = "hip"

    def linear_algo(self, dtype: torch.dtype, N: int, n_val: int, T: int, d_in: int, d_out: int,
                    semantics: int, algo: int, want_pair: bool) -> int:
        lib = load_library()
        rc = lib.gs_linear_dot_algo(_TORCH_TO_GS[dtype], N, n_val, T, d_in, d_out, semantics,
                                    algo, int(want_pair))
        _check(rc if rc < 0 else 0, "gs_linear_dot_algo")
        return rc

    def linear_dot(self, A: torch.Tensor, G: torch.Tensor, n_val: int, *, val_start=None,
                   semantics: int = SEM_PAIRWISE_SUM, algo: int = ALGO_AUTO,
                   rounding: int = ROUND_FP32, want_pair: bool = False
                   ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        dev = _require_device(A, G)
        if A.dtype != G.dtype:
            raise GhostHipError(f"A and G dtypes differ: {A.dtype} vs {G.dtype}")
        A = A.contiguous()
        G = G.contiguous()
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T:
            raise GhostHipError(f"A {tuple(A.shape)} and G {tuple(G.shape)} token counts differ")
        vs = N - n_val if val_start is None else int(val_start)
        n_t = N - n_val
        dt = _gs_dtype(A)
        lib = load_library()
        ws_bytes = lib.gs_linear_dot_workspace(dt, N, n_val, T, d_in, d_out, semantics, algo,
                                               int(want_pair))
        if ws_bytes == 0:
            raise GhostHipError(
                f"gs_linear_dot: invalid arguments N={N} n_val={n_val} T={T} d_in={d_in} "
                f"d_out={d_out} semantics={semantics} algo={algo} pair={want_pair}")
        ws = _workspace(ws_bytes, dev)
        out = torch.empty(n_t, dtype=torch.float32, device=dev)
        pair = torch.empty((n_val, n_t), dtype=torch.float32, device=dev) if want_pair else None
        rc = lib.gs_linear_dot(A.data_ptr(), G.data_ptr(), dt, N, n_val, vs, T, d_in, d_out,
                               semantics, algo, rounding, out.data_ptr(), _ptr(pair),
                               ws.data_ptr(), ws_bytes, _stream(dev))
        _check(rc, "gs_linear_dot")
        return out, pair

    def linear_dot_noalloc(self, A: torch.Tensor, G: torch.Tensor, n_val: int,
                           out: torch.Tensor, pair: Optional[torch.Tensor] = None, *,
                           val_start=None, semantics: int = SEM_PAIRWISE_SUM,
                           algo: int = ALGO_AUTO, rounding: int = ROUND_FP32) -> None:
        """gs_linear_dot_noalloc into caller-given outputs (out [n_train], pair [n_val,
        n_train] or None); nothing is allocated (A and G must be contiguous)."""
        _require_device(A, G, out, pair)
        if not (A.is_contiguous() and G.is_contiguous() and out.is_contiguous()):
            raise GhostHipError("linear_dot_noalloc: A, G and out must be contiguous")
        if A.dtype != G.dtype:
            raise GhostHipError(f"A and G dtypes differ: {A.dtype} vs {G.dtype}")
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T:
            raise GhostHipError(f"A {tuple(A.shape)} and G {tuple(G.shape)} token counts differ")
        n_t = N - n_val
        if out.dtype != torch.float32 or out.numel() != n_t or \
                (pair is not None and (pair.dtype != torch.float32 or
                                       pair.numel() != n_val * n_t)):
            raise GhostHipError("linear_dot_noalloc: outputs must be fp32 [n_train] and "
                                "[n_val, n_train]")
        vs = N - n_val if val_start is None else int(val_start)
        rc = load_library().gs_linear_dot_noalloc(
            A.data_ptr(), G.data_ptr(), _gs_dtype(A), N, n_val, vs, T, d_in, d_out, semantics,
            algo, rounding, out.data_ptr(), _ptr(pair), _stream(A.device))
        _check(rc, "gs_linear_dot_noalloc")

    def linear_val_gradient(self, A: torch.Tensor, G: torch.Tensor, n_val: int, *,
                            val_start=None, semantics: int = SEM_PAIRWISE_SUM) -> torch.Tensor:
        """The val term V [d_out, d_in] of the val-gradient algorithm (gs_linear_val_gradient):
        sum over the val rows of g a^T, or with SEM_PRESUM the product of the val rows
        presummed per token position."""
        dev = _require_device(A, G)
        if A.dtype != G.dtype:
            raise GhostHipError(f"A and G dtypes differ: {A.dtype} vs {G.dtype}")
        A = A.contiguous()
        G = G.contiguous()
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T:
            raise GhostHipError(f"A {tuple(A.shape)} and G {tuple(G.shape)} token counts differ")
        vs = N - n_val if val_start is None else int(val_start)
        dt = _gs_dtype(A)
        lib = load_library()
        ws_bytes = lib.gs_linear_val_gradient_workspace(dt, N, n_val, T, d_in, d_out, semantics)
        if ws_bytes == 0:
            raise GhostHipError(f"gs_linear_val_gradient: invalid arguments N={N} n_val={n_val} "
                                f"T={T} d_in={d_in} d_out={d_out} semantics={semantics}")
        ws = _workspace(ws_bytes, dev)
        V = torch.empty((d_out, d_in), dtype=A.dtype, device=dev)
        rc = lib.gs_linear_val_gradient(A.data_ptr(), G.data_ptr(), dt, N, n_val, vs, T, d_in,
                                        d_out, semantics, V.data_ptr(), ws.data_ptr(), ws_bytes,
                                        _stream(dev))
        _check(rc, "gs_linear_val_gradient")
        return V

    def linear_dot_train_grad(self, A: torch.Tensor, G: torch.Tensor, n_val: int, *,
                              val_start=None, semantics: int = SEM_PAIRWISE_SUM,
                              grad_scale: Optional[float] = None,
                              grad_dtype: Optional[torch.dtype] = None, bias: bool = False,
                              bias_grad_scale: Optional[float] = None,
                              bias_grad_dtype: Optional[torch.dtype] = None,
                              conv1d: bool = False):
        """Weight dots and weight train gradient in one pass over the train rows
        (gs_linear_dot_train_grad), with the bias dots and bias train gradient when `bias`;
        with conv1d the HF Conv1D form (gs_conv1d_dot_train_grad: train gradient [d_in, d_out]).
        Returns (dot, grad, bias_dot, bias_grad), entries not asked for None; None for the
        cases the kernels do not take (non-bf16, unaligned, T not a multiple of 64, feature
        counts not multiples of 8)."""
        dev = _require_device(A, G)
        if A.dtype != G.dtype:
            raise GhostHipError(f"A and G dtypes differ: {A.dtype} vs {G.dtype}")
        A = A.contiguous()
        G = G.contiguous()
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T:
            raise GhostHipError(f"A {tuple(A.shape)} and G {tuple(G.shape)} token counts differ")
        vs = N - n_val if val_start is None else int(val_start)
        dt = _gs_dtype(A)
        lib = load_library()
        name = "gs_conv1d_dot_train_grad" if conv1d else "gs_linear_dot_train_grad"
        ws_bytes = getattr(lib, name + "_workspace")(dt, N, n_val, T, d_in, d_out, semantics,
                                                     1 if bias else 0)
        if ws_bytes == 0:
            return None
        ws = _workspace(ws_bytes, dev)
        n_t = N - n_val
        dot = torch.empty(n_t, dtype=torch.float32, device=dev)
        grad = None
        if grad_scale is not None:
            grad = torch.empty((d_in, d_out) if conv1d else (d_out, d_in),
                               dtype=grad_dtype or A.dtype, device=dev)
        bdot = torch.empty(n_t, dtype=torch.float32, device=dev) if bias else None
        bgrad = None
        if bias and bias_grad_scale is not None:
            bgrad = torch.empty(d_out, dtype=bias_grad_dtype or A.dtype, device=dev)
        rc = getattr(lib, name)(
            A.data_ptr(), G.data_ptr(), dt, N, n_val, vs, T, d_in, d_out, semantics,
            dot.data_ptr(), _ptr(grad), _gs_dtype(grad) if grad is not None else DTYPE_BF16,
            float(grad_scale or 0.0), _ptr(bdot), _ptr(bgrad),
            _gs_dtype(bgrad) if bgrad is not None else DTYPE_BF16, float(bias_grad_scale or 0.0),
            ws.data_ptr(), ws_bytes, _stream(dev))
        if rc == ERR_UNSUPPORTED:
            return None
        _check(rc, name)
        return dot, grad, bdot, bgrad

    def linear_train_grad(self, A: torch.Tensor, G: torch.Tensor, n_val: int, scale: float, *,
                          val_start=None, out_dtype: Optional[torch.dtype] = None,
                          conv1d: bool = False) -> Optional[torch.Tensor]:
        """scale * sum over the train rows of g a^T as [d_out, d_in] (Linear weight), or
        a g^T as [d_in, d_out] with conv1d (gs_linear_train_grad); None for the cases the
        kernel does not take (non-bf16 operands, unaligned rows, feature counts not multiples
        of 8, operands past 2 GiB)."""
        dev = _require_device(A, G)
        if A.dtype != G.dtype:
            raise GhostHipError(f"A and G dtypes differ: {A.dtype} vs {G.dtype}")
        A = A.contiguous()
        G = G.contiguous()
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T:
            raise GhostHipError(f"A {tuple(A.shape)} and G {tuple(G.shape)} token counts differ")
        vs = N - n_val if val_start is None else int(val_start)
        dt = _gs_dtype(A)
        lib = load_library()
        ws_bytes = lib.gs_linear_train_grad_workspace(dt, N, n_val, T, d_in, d_out)
        if ws_bytes == 0:
            return None
        odt = out_dtype or A.dtype
        shape = (d_in, d_out) if conv1d else (d_out, d_in)
        out = torch.empty(shape, dtype=odt, device=dev)
        ws = _workspace(ws_bytes, dev)
        rc = lib.gs_linear_train_grad(A.data_ptr(), G.data_ptr(), dt, N, n_val, vs, T, d_in,
                                      d_out, float(scale), out.data_ptr(), _gs_dtype(out),
                                      1 if conv1d else 0, ws.data_ptr(), ws_bytes, _stream(dev))
        if rc == ERR_UNSUPPORTED:
            return None
        _check(rc, "gs_linear_train_grad")
        return out

    def linear_bias_dot(self, A: torch.Tensor, G: torch.Tensor, n_val: int, *, val_start=None,
                        semantics: int = SEM_PAIRWISE_SUM, algo: int = ALGO_AUTO,
                        rounding: int = ROUND_FP32, grad_scale: Optional[float] = None,
                        grad_dtype: Optional[torch.dtype] = None):
        """Weight and bias dots of a Linear layer (and the bias train gradient when
        grad_scale is given) in one pass over the train rows when the shape allows it (the
        val-gradient algorithm through gs_linear_bias_dot).  Otherwise None (the caller then
        uses linear_dot and bias_dot).  The val rows are [val_start, val_start + n_val)
        (default: the last n_val rows).  Returns (dot, bias_dot, bias_grad)."""
        dev = _require_device(A, G)
        if A.dtype != G.dtype or A.dtype != torch.bfloat16 or \
                semantics not in (SEM_PAIRWISE_SUM, SEM_PRESUM) or \
                (grad_dtype or G.dtype) not in (torch.bfloat16, torch.float32):
            return None
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        n_t = N - n_val
        vs = N - n_val if val_start is None else int(val_start)
        if n_t <= 0 or _tokens(G, N, d_out) != T or not 0 <= vs <= N - n_val:
            return None
        dt = _gs_dtype(A)
        lib = load_library()
        if lib.gs_linear_dot_algo(dt, N, n_val, T, d_in, d_out, semantics, algo,
                                  0) != ALGO_VALGRAD:
            return None
        ws_bytes = lib.gs_linear_bias_dot_workspace(dt, N, n_val, T, d_in, d_out, semantics)
        if ws_bytes == 0:
            return None
        A = A.contiguous()
        G = G.contiguous()
        ws = _workspace(ws_bytes, dev)
        out = torch.empty(n_t, dtype=torch.float32, device=dev)
        bout = torch.empty(n_t, dtype=torch.float32, device=dev)
        gdt = grad_dtype or G.dtype
        grad = torch.empty(d_out, dtype=gdt, device=dev) if grad_scale is not None else None
        rc = lib.gs_linear_bias_dot(A.data_ptr(), G.data_ptr(), dt, N, n_val, vs, T, d_in,
                                    d_out, semantics, out.data_ptr(), bout.data_ptr(),
                                    _ptr(grad), _TORCH_TO_GS[gdt], float(grad_scale or 0.0),
                                    ws.data_ptr(), ws_bytes, _stream(dev))
        _check(rc, "gs_linear_bias_dot")
        return out, bout, grad

    def linear_rowdot_bias(self, A: torch.Tensor, G: torch.Tensor, V: torch.Tensor, n_val: int,
                           *, val_start=None, grad_scale: Optional[float] = None,
                           grad_dtype: Optional[torch.dtype] = None):
        """gs_linear_rowdot_bias with a caller-formed V [d_out, d_in] (bf16): the weight dot
        sum_t g^T V a, the bias dot and (with grad_scale) the bias train gradient of the train
        rows in one pass.  None when the shape is outside the fused pass's limits.  Returns
        (dot, bias_dot, bias_grad)."""
        dev = _require_device(A, G, V)
        if not (A.dtype == G.dtype == V.dtype == torch.bfloat16):
            return None
        A = A.contiguous()
        G = G.contiguous()
        V = V.contiguous()
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T or tuple(V.shape) != (d_out, d_in):
            raise GhostHipError(f"shapes disagree: A {tuple(A.shape)} G {tuple(G.shape)} "
                                f"V {tuple(V.shape)}")
        vs = N - n_val if val_start is None else int(val_start)
        lib = load_library()
        ws_bytes = lib.gs_linear_rowdot_bias_workspace(DTYPE_BF16, N, n_val, T, d_in, d_out)
        if ws_bytes == 0:
            return None
        ws = _workspace(ws_bytes, dev)
        n_t = N - n_val
        out = torch.empty(n_t, dtype=torch.float32, device=dev)
        bout = torch.empty(n_t, dtype=torch.float32, device=dev)
        gdt = grad_dtype or G.dtype
        grad = torch.empty(d_out, dtype=gdt, device=dev) if grad_scale is not None else None
        rc = lib.gs_linear_rowdot_bias(A.data_ptr(), G.data_ptr(), V.data_ptr(), DTYPE_BF16, N,
                                       n_val, vs, T, d_in, d_out, out.data_ptr(), bout.data_ptr(),
                                       _ptr(grad), _TORCH_TO_GS[gdt], float(grad_scale or 0.0),
                                       ws.data_ptr(), ws_bytes, _stream(dev))
        _check(rc, "gs_linear_rowdot_bias")
        return out, bout, grad

    def linear_rowdot(self, A: torch.Tensor, G: torch.Tensor, V: torch.Tensor, n_val: int, *,
                      val_start=None) -> torch.Tensor:
        """dot_i = sum_t g_it^T V a_it over the train rows, V: [d_out, d_in]."""
        dev = _require_device(A, G, V)
        if not (A.dtype == G.dtype == V.dtype):
            raise GhostHipError(f"A, G, V dtypes differ: {A.dtype} {G.dtype} {V.dtype}")
        A = A.contiguous()
        G = G.contiguous()
        V = V.contiguous()
        N = A.shape[0]
        d_in, d_out = A.shape[-1], G.shape[-1]
        T = _tokens(A, N, d_in)
        if _tokens(G, N, d_out) != T or tuple(V.shape) != (d_out, d_in):
            raise GhostHipError(f"shapes disagree: A {tuple(A.shape)} G {tuple(G.shape)} "
                                f"V {tuple(V.shape)}")
        vs = N - n_val if val_start is None else int(val_start)
        dt = _gs_dtype(A)
        lib = load_library()
        ws_bytes = lib.gs_linear_rowdot_workspace(dt, N, n_val, T, d_in, d_out)
        if ws_bytes == 0:
            raise GhostHipError(f"gs_linear_rowdot: invalid arguments N={N} n_val={n_val} T={T}")
        ws = _workspace(ws_bytes, dev)
        out = torch.empty(N - n_val, dtype=torch.float32, device=dev)
        rc = lib.gs_linear_rowdot(A.data_ptr(), G.data_ptr(), V.data_ptr(), dt, N, n_val, vs, T,
                                  d_in, d_out, out.data_ptr(), ws.data_ptr(), ws_bytes,
                                  _stream(dev))
        _check(rc, "gs_linear_rowdot")
        return out

    def bias_dot(self, G: torch.Tensor, n_val: int, *, val_start=None,
                 grad_scale: Optional[float] = None, grad_dtype: Optional[torch.dtype] = None
                 ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        dev = _require_device(G)
        G = G.contiguous()
        N, d = G.shape[0], G.shape[-1]
        T = _tokens(G, N, d)
        vs = N - n_val if val_start is None else int(val_start)
        lib = load_library()
        ws_bytes = lib.gs_bias_dot_workspace(N, T, d)
        ws = _workspace(ws_bytes, dev)
        out = torch.empty(N - n_val, dtype=torch.float32, device=dev)
        grad = None
        if grad_scale is not None:
            grad = torch.empty(d, dtype=grad_dtype or G.dtype, device=dev)
        gdt = _gs_dtype(grad) if grad is not None else DTYPE_F32
        rc = lib.gs_bias_dot(G.data_ptr(), _gs_dtype(G), N, n_val, vs, T, d, out.data_ptr(),
                             _ptr(grad), gdt, float(grad_scale or 0.0), ws.data_ptr(), ws_bytes,
                             _stream(dev))
        _check(rc, "gs_bias_dot")
        return out, grad

    def embedding_dot(self, ids: torch.Tensor, G: torch.Tensor, n_val: int, vocab: int, *,
                      val_start=None) -> torch.Tensor:
        dev = _require_device(ids, G)
        ids = ids.to(torch.int64).contiguous()
        G = G.contiguous()
        N, d = G.shape[0], G.shape[-1]
        T = ids.numel() // N
        if _tokens(G, N, d) != T:
            raise GhostHipError(f"ids {tuple(ids.shape)} and G {tuple(G.shape)} disagree")
        vs = N - n_val if val_start is None else int(val_start)
        lib = load_library()
        ws_bytes = lib.gs_embedding_dot_workspace(N, n_val, T, d, vocab)
        if ws_bytes == 0:
            raise GhostHipError(f"gs_embedding_dot: invalid arguments N={N} n_val={n_val}")
        ws = _workspace(ws_bytes, dev)
        out = torch.empty(N - n_val, dtype=torch.float32, device=dev)
        rc = lib.gs_embedding_dot(ids.data_ptr(), G.data_ptr(), _gs_dtype(G), N, n_val, vs, T, d,
                                  vocab, out.data_ptr(), ws.data_ptr(), ws_bytes, _stream(dev))
        _check(rc, "gs_embedding_dot")
        return out

    def embedding_train_grad(self, ids: torch.Tensor, G: torch.Tensor, n_val: int,
                             scale: float, out: torch.Tensor, *, accumulate: bool = False,
                             val_start=None) -> None:
        """out[v] (+)= scale * sum of the train rows of G whose token id is v
        (gs_embedding_train_grad); out: [vocab, d] bf16 or fp32, written in place."""
        dev = _require_device(ids, G, out)
        ids = ids.to(torch.int64).contiguous()
        G = G.contiguous()
        N, d = G.shape[0], G.shape[-1]
        T = ids.numel() // N
        if _tokens(G, N, d) != T or out.dim() != 2 or out.shape[1] != d or \
                not out.is_contiguous():
            raise GhostHipError(f"embedding_train_grad: ids {tuple(ids.shape)}, G "
                                f"{tuple(G.shape)} and out {tuple(out.shape)} disagree")
        vocab = out.shape[0]
        vs = N - n_val if val_start is None else int(val_start)
        lib = load_library()
        ws_bytes = lib.gs_embedding_train_grad_workspace(N, n_val, T, d, vocab)
        if ws_bytes == 0:
            raise GhostHipError(f"gs_embedding_train_grad: invalid arguments N={N} n_val={n_val}")
        ws = _workspace(ws_bytes, dev)
        rc = lib.gs_embedding_train_grad(ids.data_ptr(), G.data_ptr(), _gs_dtype(G), N, n_val,
                                         vs, T, d, vocab, float(scale), out.data_ptr(),
                                         _gs_dtype(out), int(accumulate), ws.data_ptr(),
                                         ws_bytes, _stream(dev))
        _check(rc, "gs_embedding_train_grad")

    def layernorm_dot(self, X: torch.Tensor, G: torch.Tensor, n_val: int, eps: float, *,
                      val_start=None, want_dot: bool = True, want_bias: bool = True,
                      grad_scale: Optional[float] = None,
                      grad_dtype: Optional[torch.dtype] = None):
        """Returns (dot_w, dot_b, grad_w, grad_b); entries not asked for are None."""
        dev = _require_device(X, G)
        if X.dtype != G.dtype:
            raise GhostHipError(f"X and G dtypes differ: {X.dtype} vs {G.dtype}")
        X = X.contiguous()
        G = G.contiguous()
        N, F = X.shape[0], X.shape[-1]
        T = _tokens(X, N, F)
        vs = N - n_val if val_start is None else int(val_start)
        lib = load_library()
        ws_bytes = lib.gs_layernorm_dot_workspace(N, T, F)
        ws = _workspace(ws_bytes, dev)
        n_t = N - n_val
        dw = torch.empty(n_t, dtype=torch.float32, device=dev) if want_dot else None
        db = torch.empty(n_t, dtype=torch.float32, device=dev) if (want_dot and want_bias) else None
        gw = gb = None
        gdt = grad_dtype or X.dtype
        if grad_scale is not None:
            gw = torch.empty(F, dtype=gdt, device=dev)
            gb = torch.empty(F, dtype=gdt, device=dev) if want_bias else None
        rc = lib.gs_layernorm_dot(X.data_ptr(), G.data_ptr(), _gs_dtype(X), N, n_val, vs, T, F,
                                  float(eps), _ptr(dw), _ptr(db), _ptr(gw), _ptr(gb),
                                  _TORCH_TO_GS[gdt], float(grad_scale or 0.0), ws.data_ptr(),
                                  ws_bytes, _stream(dev))
        _check(rc, "gs_layernorm_dot")
        return dw, db, gw, gb

    def kron_proj(self, A: torch.Tensor, G: torch.Tensor, P_i: torch.Tensor, P_o: torch.Tensor,
                  scale: float, *, layout: int = PROJ_KO_KI,
                  out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        dev = _require_device(A, G, P_i, P_o)
        if A.dtype != G.dtype:
            raise GhostHipError(f"A and G dtypes differ: {A.dtype} vs {G.dtype}")
        A = A.contiguous()
        G = G.contiguous()
        P_i = P_i.to(A.dtype).contiguous()
        P_o = P_o.to(A.dtype).contiguous()
        B = A.shape[0]
        n_a, n_g = A.shape[-1], G.shape[-1]
        T = A.numel() // (B * n_a)
        if G.numel() // (B * n_g) != T:
            raise GhostHipError(f"A {tuple(A.shape)} and G {tuple(G.shape)} token counts differ")
        k_i, k_o = P_i.shape[0], P_o.shape[0]
        if layout == PROJ_KO_KI:
            if P_i.shape[1] != n_a or P_o.shape[1] != n_g:
                raise GhostHipError("projection widths do not match the layer")
            shape = (B, k_o, k_i)
        else:
            if P_i.shape[1] != n_g or P_o.shape[1] != n_a:
                raise GhostHipError("projection widths do not match the layer (Conv1D roles)")
            shape = (B, k_i, k_o)
        lib = load_library()
        ws_bytes = lib.gs_kron_proj_workspace(B, T, k_i, k_o)
        ws = _workspace(ws_bytes, dev)
        out = torch.empty(shape, dtype=out_dtype, device=dev)
        rc = lib.gs_kron_proj(A.data_ptr(), G.data_ptr(), _gs_dtype(A), B, T, n_a, n_g,
                              P_i.data_ptr(), P_o.data_ptr(), _gs_dtype(P_i), k_i, k_o, layout,
                              float(scale), out.data_ptr(), _TORCH_TO_GS[out_dtype],
                              ws.data_ptr(), ws_bytes, _stream(dev))
        _check(rc, "gs_kron_proj")
        return out

    def kron_embed_proj(self, ids: torch.Tensor, G: torch.Tensor, P_iT: torch.Tensor,
                        P_o: torch.Tensor, scale: float = 1.0, *,
                        out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """out[b] = scale * sum_t (P_o g_bt)(P_iT[ids_bt])^T, [B, k_o, k_i]."""
        dev = _require_device(ids, G, P_iT, P_o)
        B = ids.shape[0]
        ids = ids.reshape(B, -1).long().contiguous()
        T = ids.shape[1]
        n_g = G.shape[-1]
        if G.numel() != B * T * n_g:
            raise GhostHipError(f"ids {tuple(ids.shape)} and G {tuple(G.shape)} disagree")
        G = G.contiguous()
        P_iT = P_iT.to(G.dtype).contiguous()
        P_o = P_o.to(G.dtype).contiguous()
        vocab, k_i = P_iT.shape
        k_o = P_o.shape[0]
        if P_o.shape[1] != n_g:
            raise GhostHipError("P_o width does not match the embedding dimension")
        lib = load_library()
        ws_bytes = lib.gs_kron_proj_workspace(B, T, k_i, k_o)
        ws = _workspace(ws_bytes, dev)
        out = torch.empty((B, k_o, k_i), dtype=out_dtype, device=dev)
        rc = lib.gs_kron_embed_proj(ids.data_ptr(), G.data_ptr(), _gs_dtype(G), B, T, n_g,
                                    P_iT.data_ptr(), P_o.data_ptr(), _gs_dtype(P_iT), vocab, k_i,
                                    k_o, float(scale), out.data_ptr(), _TORCH_TO_GS[out_dtype],
                                    ws.data_ptr(), ws_bytes, _stream(dev))
        _check(rc, "gs_kron_embed_proj")
        return out


    def ordered_sum_(self, tensors) -> torch.Tensor:
        """tensors[0] += tensors[1], then += tensors[2], ... in order, in place, in one launch
        per 48 tensors: fp32 arithmetic, each partial sum rounded to tensors[0]'s dtype (the
        in-place adds' own rounding).  Every tensor: contiguous, bf16 or fp32, the same
        number of elements, on one device.  Returns tensors[0]."""
        total = tensors[0]
        dev = _require_device(*tensors)
        n = total.numel()
        for t in tensors:
            if t.numel() != n or not t.is_contiguous() or \
                    t.dtype not in (torch.bfloat16, torch.float32):
                raise GhostHipError("ordered_sum_: contiguous bf16 / fp32 tensors of one size")
        k = len(tensors)
        ptrs = (ctypes.c_void_p * k)(*[t.data_ptr() for t in tensors])
        dts = (ctypes.c_int * k)(*[_TORCH_TO_GS[t.dtype] for t in tensors])
        rc = load_library().gs_ordered_sum(ptrs, dts, k, n, total.data_ptr(),
                                           _TORCH_TO_GS[total.dtype], _stream(dev))
        _check(rc, "gs_ordered_sum")
        return total


_backend = None


def ops():
    """The active kernel layer (the HIP library unless a test installed a checker)."""
    global _backend
    if _backend is None:
        _backend = HipOps()
    return _backend


def _install_backend(backend) -> None:
    """Test seam: replace the kernel layer (host-logic tests on machines without a GPU)."""
    global _backend
    _backend = backend
