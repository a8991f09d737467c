"""The HIP samplers and the engine on the GPU against outputs of the reference's own
functions (tests/golden/reference_vectors.pt, written by tests/golden/make_golden.py).

Tolerances: 2e-2 normwise where the reference rounds through bf16 (its ghost branch, the
embedding and LayerNorm dots, every bf16 input), 1e-4 where it computes in fp32 (the
materialised branch and the bias dot on fp32 inputs, train gradients and weights of an fp32
model).
"""
import os

import pytest
import torch
from torch import nn

from ghostsuite_amd import GradDotProdEngine
from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
from tests.helpers import BF16_TOL, FP32_TOL, assert_close

pytestmark = pytest.mark.gpu

VECTORS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                       "reference_vectors.pt")


@pytest.fixture(scope="module")
def golden():
    return torch.load(VECTORS, weights_only=True)


@pytest.fixture(autouse=True)
def _reset_options():
    saved = dict(S.options)
    yield
    S.options.clear()
    S.options.update(saved)


def _tol(c, bf16_rounded):
    return BF16_TOL if bf16_rounded or c["A" if "A" in c else "B"].dtype == torch.bfloat16 \
        else FP32_TOL


def test_linear_samplers_match_reference_outputs(gpu, golden):
    for name, c in golden["samplers"].items():
        if not name.startswith("linear_"):
            continue
        ghost = "_ghost_" in name
        print(f"golden {name}", flush=True)
        lin = nn.Linear(c["A"].shape[-1], c["B"].shape[-1]).to(gpu, c["A"].dtype)
        lin.use_ghost_computation = ghost
        S._compute_linear_dot_product(lin, c["A"].to(gpu), c["B"].to(gpu), c["n_val"])
        torch.cuda.synchronize()
        assert_close(lin.weight.grad_dot_prod.cpu(), c["dot"], _tol(c, ghost), f"{name} dot")
        assert_close(lin.bias.grad_dot_prod.cpu(), c["bias_dot"], _tol(c, False),
                     f"{name} bias")
        assert lin.weight.grad_dot_prod.dtype == c["dot"].dtype, name
        assert lin.bias.grad_dot_prod.dtype == c["bias_dot"].dtype, name


def test_embedding_layernorm_conv1d_samplers_match_reference_outputs(gpu, golden):
    for name, c in golden["samplers"].items():
        print(f"golden {name}", flush=True)
        if name.startswith("embedding_"):
            emb = nn.Embedding(c["vocab"], c["B"].shape[-1]).to(gpu)
            S._compute_embedding_dot_product(emb, c["ids"].to(gpu), c["B"].to(gpu), c["n_val"])
            torch.cuda.synchronize()
            assert_close(emb.weight.grad_dot_prod.cpu(), c["dot"], BF16_TOL, name)
            assert emb.weight.grad_dot_prod.dtype == c["dot"].dtype, name
        elif name.startswith("layernorm_"):
            ln = nn.LayerNorm(c["A"].shape[-1], eps=c["eps"]).to(gpu, c["A"].dtype)
            S._compute_layernorm_dot_product(ln, c["A"].to(gpu), c["B"].to(gpu), c["n_val"])
            torch.cuda.synchronize()
            assert_close(ln.weight.grad_dot_prod.cpu(), c["dot"], BF16_TOL, f"{name} w")
            assert_close(ln.bias.grad_dot_prod.cpu(), c["bias_dot"], BF16_TOL, f"{name} b")
            assert ln.weight.grad_dot_prod.dtype == c["dot"].dtype, name
            assert ln.bias.grad_dot_prod.dtype == c["bias_dot"].dtype, name
        elif name.startswith("conv1d_"):
            transformers = pytest.importorskip("transformers")
            conv = transformers.pytorch_utils.Conv1D(c["B"].shape[-1], c["A"].shape[-1])
            conv = conv.to(gpu, c["A"].dtype)
            conv.use_ghost_computation = "_ghost_" in name
            S._compute_Conv1D_dot_product(conv, c["A"].to(gpu), c["B"].to(gpu), c["n_val"])
            torch.cuda.synchronize()
            assert_close(conv.weight.grad_dot_prod.cpu(), c["dot"], BF16_TOL, f"{name} dot")
            assert_close(conv.bias.grad_dot_prod.cpu(), c["bias_dot"], BF16_TOL,
                         f"{name} bias")
            assert conv.weight.grad_dot_prod.dtype == c["dot"].dtype, name
            assert conv.bias.grad_dot_prod.dtype == c["bias_dot"].dtype, name


def test_engine_on_gpu_matches_reference_engine(gpu, golden):
    """The tied model of the golden file, two SGD steps through this package's engine with
    the HIP kernels: per-parameter dots, logged aggregates, .grad and final weights."""
    from tests.golden.make_golden import tied_net_state
    g = golden["engine_tied"]
    net = tied_net_state().to(gpu)
    X, Y, n_v = g["X"].to(gpu), g["Y"].to(gpu), g["n_val"]
    n_t = X.shape[0] - n_v
    opt = torch.optim.SGD(net.parameters(), lr=g["lr"])
    eng = GradDotProdEngine(net, val_batch_size=n_v, use_dummy_bias=False)
    eng.attach(opt)
    for it, want in enumerate(g["steps"]):
        print(f"golden engine step {it}", flush=True)
        eng.attach_train_batch(X[:n_t], Y[:n_t], it, it)
        loss = torch.nn.functional.cross_entropy(net(X).reshape(-1, 13), Y.reshape(-1))
        opt.zero_grad()
        loss.backward()
        torch.cuda.synchronize()
        dots = {n: p.grad_dot_prod.cpu() for n, p in net.named_parameters()
                if hasattr(p, "grad_dot_prod")}
        assert sorted(dots) == sorted(want["dots"])
        for n in dots:
            assert_close(dots[n], want["dots"][n], BF16_TOL, f"step {it} dot {n}")
        eng.prepare_gradients()
        for n, p in net.named_parameters():
            assert_close(p.grad.cpu(), want["grads"][n], FP32_TOL, f"step {it} grad {n}")
        opt.step()
        eng.aggregate_and_log()
        eng.clear_gradients()
        assert_close(eng.dot_product_log[-1]["dot_product"], want["logged"], BF16_TOL,
                     f"step {it} logged")
    eng.detach()
    for k, v in net.state_dict().items():
        assert_close(v.cpu(), g["final"][k], FP32_TOL, f"final {k}")
