"""CPU stand-in for the kernel layer, used only by host-logic tests (routing, hooks, engine
state machine) on machines without a GPU.  Every op is the oracle's float64 closed form,
so these tests check what the engines do with the results, not the kernels."""
import torch

from ghostsuite_amd import _native
from oracle import ghost_ref as R


class OracleOps:
    name = "oracle"

    def __init__(self):
        self.calls = []

    def linear_algo(self, dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair):
        return _native.ALGO_GHOST if algo in (_native.ALGO_AUTO, _native.ALGO_GHOST) else algo

    def linear_dot(self, A, G, n_val, *, val_start=None, semantics=0, algo=0, rounding=0,
                   want_pair=False):
        self.calls.append(("linear_dot", tuple(A.shape), tuple(G.shape), semantics))
        sem = "pairwise" if semantics == _native.SEM_PAIRWISE_SUM else "presum"
        dot = R.linear_dot_exact(A.float(), G.float(), n_val, sem, val_start=val_start).float()
        pair = None
        if want_pair:
            pair = R.linear_dot_exact(A.float(), G.float(), n_val, sem, val_start=val_start,
                                      pair=True).float()
        return dot.to(A.device), pair

    def linear_bias_dot(self, A, G, n_val, *, semantics=0, algo=0, rounding=0, grad_scale=None,
                        grad_dtype=None):
        """The fused weight + bias pass, as closed forms."""
        self.calls.append(("linear_bias_dot", tuple(A.shape), tuple(G.shape)))
        dot, _ = self.linear_dot(A, G, n_val, semantics=semantics)
        bdot, grad = self.bias_dot(G, n_val, grad_scale=grad_scale, grad_dtype=grad_dtype)
        return dot, bdot, grad

    def linear_dot_train_grad(self, A, G, n_val, *, val_start=None, semantics=0,
                              grad_scale=None, grad_dtype=None, bias=False,
                              bias_grad_scale=None, bias_grad_dtype=None):
        """The fused weight dot + train gradient (+ bias dot and gradient), as closed forms."""
        self.calls.append(("linear_dot_train_grad", tuple(A.shape), tuple(G.shape)))
        dot, _ = self.linear_dot(A, G, n_val, val_start=val_start, semantics=semantics)
        grad = None
        if grad_scale is not None:
            grad = self.linear_train_grad(A, G, n_val, grad_scale, val_start=val_start,
                                          out_dtype=grad_dtype)
        bdot = bgrad = None
        if bias:
            bdot, bgrad = self.bias_dot(G, n_val, val_start=val_start,
                                        grad_scale=bias_grad_scale, grad_dtype=bias_grad_dtype)
        return dot, grad, bdot, bgrad

    def linear_train_grad(self, A, G, n_val, scale, *, val_start=None, out_dtype=None,
                          conv1d=False):
        self.calls.append(("linear_train_grad", tuple(A.shape), tuple(G.shape)))
        N = A.shape[0]
        a, _ = R.split_rows(A.double().reshape(N, -1, A.shape[-1]), n_val, val_start)
        g, _ = R.split_rows(G.double().reshape(N, -1, G.shape[-1]), n_val, val_start)
        a, g = a.reshape(-1, a.shape[-1]), g.reshape(-1, g.shape[-1])
        w = (a.t() @ g) if conv1d else (g.t() @ a)
        return (w * scale).to(out_dtype or A.dtype)

    def bias_dot(self, G, n_val, *, val_start=None, grad_scale=None, grad_dtype=None):
        self.calls.append(("bias_dot", tuple(G.shape)))
        dot = R.bias_dot_exact(G.float(), n_val, val_start).float()
        grad = None
        if grad_scale is not None:
            N, d = G.shape[0], G.shape[-1]
            tr, _ = R.split_rows(G.double().reshape(N, -1, d), n_val, val_start)
            grad = (tr.sum((0, 1)) * grad_scale).to(grad_dtype or G.dtype)
        return dot, grad

    def embedding_dot(self, ids, G, n_val, vocab, *, val_start=None):
        self.calls.append(("embedding_dot", tuple(G.shape)))
        return R.embedding_dot_exact(ids, G.float(), n_val, val_start).float()

    def embedding_train_grad(self, ids, G, n_val, scale, out, *, accumulate=False,
                             val_start=None):
        self.calls.append(("embedding_train_grad", tuple(G.shape)))
        N, d = G.shape[0], G.shape[-1]
        tr_i, _ = R.split_rows(ids.reshape(N, -1).long(), n_val, val_start)
        tr_g, _ = R.split_rows(G.double().reshape(N, -1, d), n_val, val_start)
        g = torch.zeros(out.shape, dtype=torch.float64)
        g.index_add_(0, tr_i.reshape(-1), tr_g.reshape(-1, d))
        g *= scale
        if accumulate:
            touched = torch.zeros(out.shape[0], dtype=torch.bool)
            touched[tr_i.reshape(-1)] = True
            out[touched] = (out[touched].double() + g[touched]).to(out.dtype)
        else:
            out.copy_(g.to(out.dtype))

    def layernorm_dot(self, X, G, n_val, eps, *, val_start=None, want_dot=True, want_bias=True,
                      grad_scale=None, grad_dtype=None):
        self.calls.append(("layernorm_dot", tuple(X.shape)))
        dw = db = gw = gb = None
        if want_dot:
            w, b = R.layernorm_dot_exact(X.float(), G.float(), n_val, eps, val_start)
            dw = w.float()
            db = b.float() if want_bias else None
        if grad_scale is not None:
            N, Fd = X.shape[0], X.shape[-1]
            x = X.double().reshape(N, -1, Fd)
            g = G.double().reshape(N, -1, Fd)
            xh = torch.nn.functional.layer_norm(x, (Fd,), eps=eps)
            tw, _ = R.split_rows((g * xh).sum(1), n_val, val_start)
            tb, _ = R.split_rows(g.sum(1), n_val, val_start)
            gw = (tw.sum(0) * grad_scale).to(grad_dtype or X.dtype)
            gb = (tb.sum(0) * grad_scale).to(grad_dtype or X.dtype) if want_bias else None
        return dw, db, gw, gb

    def kron_proj(self, A, G, P_i, P_o, scale, *, layout=0, out_dtype=torch.float32):
        self.calls.append(("kron_proj", tuple(A.shape)))
        out = R.kron_proj_exact(A.float(), G.float(), P_i.float(), P_o.float(), scale,
                                conv1d=layout == _native.PROJ_KI_KO)
        return out.to(out_dtype)

    def kron_embed_proj(self, ids, G, P_iT, P_o, scale=1.0, *, out_dtype=torch.float32):
        self.calls.append(("kron_embed_proj", tuple(G.shape)))
        out = R.kron_embed_proj_exact(ids, G.float(), P_iT.t().float(), P_o.float(), scale)
        return out.to(out_dtype)


class use_oracle_backend:
    """Context manager installing OracleOps as the kernel layer."""

    def __enter__(self):
        self.ops = OracleOps()
        _native._install_backend(self.ops)
        return self.ops

    def __exit__(self, *exc):
        _native._install_backend(None)
        return False
