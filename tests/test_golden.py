"""The oracle and the host logic against vectors written by the reference's own functions
(tests/golden/make_golden.py; inputs and outputs only, loaded with weights_only=True).

  - the oracle's reference op sequences (*_ref) reproduce the reference's bf16 rounding
    sequence bit for bit on the same inputs (CPU, one thread, the torch build the vectors
    were written with; a later torch release may move a last bit, and the check then
    degrades to one bf16 step per entry, reported in the assertion);
  - the exact closed forms sit within the bf16 tolerance of the reference's outputs (2e-2
    normwise) and within 1e-5 where the reference computes in fp32;
  - the engine's routing, aggregation and tied-weight overwrite match the reference
    engine's over two SGD steps (the kernel layer here is the oracle's CPU stand-in);
  - the Gaussian projection matrices equal the reference's on the CPU generator.
"""
import os

import pytest
import torch

from oracle import ghost_ref as R
from tests.helpers import BF16_TOL, assert_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
VECTORS = os.path.join(HERE, "reference_vectors.pt")


@pytest.fixture(scope="module")
def golden():
    return torch.load(VECTORS, weights_only=True)


def _bitwise_or_one_step(got, want, what):
    """Equal bits, else every entry within one bf16 rounding step (2^-8 relative)."""
    got = got.float()
    want = want.float()
    if torch.equal(got, want):
        return
    rel = ((got - want).abs() / want.abs().clamp_min(1e-30)).max().item()
    assert rel <= 2.0 ** -8, f"{what}: not bit-equal, worst relative difference {rel:.3e}"


def _cases(golden, prefix):
    return {k: v for k, v in golden["samplers"].items() if k.startswith(prefix)}


def test_vectors_present_and_from_the_reference(golden):
    meta = golden["meta"]
    assert set(meta["sha256"]) >= {"ghostEngines/supported_layers_grad_samplers_dotprod.py",
                                   "ghostEngines/graddotprod_engine.py"}
    assert len(golden["samplers"]) == 24 and len(golden["projection"]) == 3


def test_linear_reference_sequence_bits(golden):
    torch.set_num_threads(1)
    for name, c in _cases(golden, "linear_").items():
        ghost = "_ghost_" in name
        w, b = R.linear_dot_ref(c["A"], c["B"], c["n_val"], use_ghost=ghost)
        _bitwise_or_one_step(w, c["dot"], f"{name} weight")
        _bitwise_or_one_step(b, c["bias_dot"], f"{name} bias")
        sem = "pairwise" if ghost else "presum"
        tol = BF16_TOL if (ghost or c["A"].dtype == torch.bfloat16) else 1e-5
        assert_close(R.linear_dot_exact(c["A"], c["B"], c["n_val"], sem), c["dot"], tol,
                     f"{name} exact")
        assert_close(R.bias_dot_exact(c["B"], c["n_val"]), c["bias_dot"],
                     BF16_TOL if c["B"].dtype == torch.bfloat16 else 1e-5, f"{name} bias exact")


def test_conv2d_reference_sequence_bits(golden):
    """The reference's Conv2d materialised branch (all bf16) against conv2d_dot_ref bit for
    bit, and the float64 presum form within the bf16 tolerance."""
    torch.set_num_threads(1)
    cases = _cases(golden, "conv2d_")
    assert sorted(cases) == ["conv2d_mat_bf16", "conv2d_mat_fp32"]
    for name, c in cases.items():
        conv = {k: c[k] for k in ("kernel_size", "padding", "stride", "dilation")}
        w, b = R.conv2d_dot_ref(c["A"], c["B"], c["n_val"], conv)
        _bitwise_or_one_step(w, c["dot"], f"{name} weight")
        _bitwise_or_one_step(b, c["bias_dot"], f"{name} bias")
        assert_close(R.conv2d_dot_exact(c["A"], c["B"], c["n_val"], conv), c["dot"], BF16_TOL,
                     f"{name} exact")


def test_embedding_reference_sequence_bits(golden):
    torch.set_num_threads(1)
    for name, c in _cases(golden, "embedding_").items():
        got = R.embedding_dot_ref(c["ids"], c["B"], c["n_val"], c["vocab"])
        _bitwise_or_one_step(got, c["dot"], name)
        assert_close(R.embedding_dot_exact(c["ids"], c["B"], c["n_val"]), c["dot"], BF16_TOL,
                     f"{name} exact")


def test_layernorm_reference_sequence_bits(golden):
    torch.set_num_threads(1)
    for name, c in _cases(golden, "layernorm_").items():
        w, b = R.layernorm_dot_ref(c["A"], c["B"], c["n_val"], c["eps"])
        _bitwise_or_one_step(w, c["dot"], f"{name} weight")
        _bitwise_or_one_step(b, c["bias_dot"], f"{name} bias")
        ew, eb = R.layernorm_dot_exact(c["A"], c["B"], c["n_val"], c["eps"])
        assert_close(ew, c["dot"], BF16_TOL, f"{name} exact weight")
        assert_close(eb, c["bias_dot"], BF16_TOL, f"{name} exact bias")


def test_conv1d_reference_sequence_bits(golden):
    torch.set_num_threads(1)
    cases = _cases(golden, "conv1d_")
    if not cases:
        pytest.skip("vectors written without transformers")
    for name, c in cases.items():
        w, b = R.conv1d_dot_ref(c["A"], c["B"], c["n_val"], use_ghost="_ghost_" in name)
        _bitwise_or_one_step(w, c["dot"], f"{name} weight")
        _bitwise_or_one_step(b, c["bias_dot"], f"{name} bias")
        assert_close(R.linear_dot_exact(c["A"], c["B"], c["n_val"], "presum"), c["dot"],
                     BF16_TOL, f"{name} exact")


def test_planted_rounding_mistake_is_caught(golden):
    """Dropping the bf16 rounding of the Gram products (fp32 matmuls in place of bf16 ones)
    changes the bits of the reference sequence's output."""
    c = golden["samplers"]["linear_ghost_3d_fp32"]
    A, B, n_val = c["A"], c["B"], c["n_val"]
    n_t = A.shape[0] - n_val
    a = A.to(torch.bfloat16).float()
    b = B.to(torch.bfloat16).float()
    a_dot = a[:n_t].reshape(-1, a.shape[-1]) @ a[n_t:].reshape(-1, a.shape[-1]).T
    b_dot = b[:n_t].reshape(-1, b.shape[-1]) @ b[n_t:].reshape(-1, b.shape[-1]).T
    wrong = (a_dot * b_dot).sum(1).reshape(n_t, -1).sum(1)
    assert not torch.equal(wrong, c["dot"])


def test_projection_matrices_equal_reference(golden):
    from ghostsuite_amd.gradProjection.projection_utils import init_projection_matrix_gaussian
    for name, c in golden["projection"].items():
        P = init_projection_matrix_gaussian(c["rows"], c["cols"], dtype=torch.float32,
                                            device=torch.device("cpu"), seed=c["seed"])
        assert torch.equal(P, c["P"]), name


def test_engine_routing_matches_reference_engine(golden):
    """TiedNet (Embedding -> LayerNorm -> Linear -> tanh -> Linear tied to the Embedding),
    4 train + 2 val rows, two SGD steps in the reference's step order, through this
    package's engine on the oracle's CPU kernel layer: the same parameters carry dots (the
    Embedding's replaces the tied Linear's), the logged aggregate, .grad and the weights
    after each step."""
    from ghostsuite_amd import GradDotProdEngine
    from tests.golden.make_golden import tied_net_state
    from tests.oracle_backend import use_oracle_backend
    g = golden["engine_tied"]
    net = tied_net_state()
    for k, v in net.state_dict().items():
        assert torch.equal(v, g["init"][k]), k
    X, Y, n_v = g["X"], g["Y"], g["n_val"]
    n_t = X.shape[0] - n_v
    opt = torch.optim.SGD(net.parameters(), lr=g["lr"])
    with use_oracle_backend():
        eng = GradDotProdEngine(net, val_batch_size=n_v, use_dummy_bias=False)
        eng.attach(opt)
        for it, want in enumerate(g["steps"]):
            eng.attach_train_batch(X[:n_t], Y[:n_t], it, it)
            loss = torch.nn.functional.cross_entropy(net(X).reshape(-1, 13), Y.reshape(-1))
            opt.zero_grad()
            loss.backward()
            dots = {n: p.grad_dot_prod.detach().clone() for n, p in net.named_parameters()
                    if hasattr(p, "grad_dot_prod")}
            assert sorted(dots) == sorted(want["dots"]), (sorted(dots), sorted(want["dots"]))
            for n in dots:
                assert_close(dots[n], want["dots"][n], BF16_TOL, f"step {it} dot {n}")
            eng.prepare_gradients()
            for n, p in net.named_parameters():
                assert_close(p.grad, want["grads"][n], 1e-5, f"step {it} grad {n}")
            opt.step()
            eng.aggregate_and_log()
            eng.clear_gradients()
            assert_close(eng.dot_product_log[-1]["dot_product"], want["logged"], BF16_TOL,
                         f"step {it} logged")
        eng.detach()
    for k, v in net.state_dict().items():
        assert_close(v, g["final"][k], 1e-5, f"final {k}")


def test_sampler_dot_dtypes_match_reference_outputs(golden):
    """The dtype of every grad_dot_prod the samplers set equals the dtype of the reference's
    own output for the same layer and inputs (the golden vectors): fp32 from the ghost
    branches, Embedding and LayerNorm, the operands' dtype from Linear's materialised branch
    and bias, bf16 from Conv1D's materialised branch and bias and from Conv2d even on fp32
    inputs (those samplers cast to bf16 first).  The values come from the oracle backend
    here; the GPU golden test checks the HIP path's dtypes and values."""
    from torch import nn
    from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
    from tests.oracle_backend import use_oracle_backend
    checked = 0
    with use_oracle_backend():
        for name, c in golden["samplers"].items():
            if name.startswith("linear_"):
                layer = nn.Linear(c["A"].shape[-1], c["B"].shape[-1]).to(c["A"].dtype)
                layer.use_ghost_computation = "_ghost_" in name
                S._compute_linear_dot_product(layer, c["A"], c["B"], c["n_val"])
            elif name.startswith("conv1d_"):
                from transformers.pytorch_utils import Conv1D
                layer = Conv1D(c["B"].shape[-1], c["A"].shape[-1]).to(c["A"].dtype)
                layer.use_ghost_computation = "_ghost_" in name
                S._compute_Conv1D_dot_product(layer, c["A"], c["B"], c["n_val"])
            elif name.startswith("conv2d_"):
                layer = nn.Conv2d(c["A"].shape[1], c["B"].shape[1], c["kernel_size"],
                                  stride=c["stride"], padding=c["padding"],
                                  dilation=c["dilation"]).to(c["A"].dtype)
                S._compute_conv2d_dot_product(layer, c["A"], c["B"], c["n_val"])
            elif name.startswith("embedding_"):
                layer = nn.Embedding(c["vocab"], c["B"].shape[-1]).to(c["B"].dtype)
                S._compute_embedding_dot_product(layer, c["ids"], c["B"], c["n_val"])
            elif name.startswith("layernorm_"):
                layer = nn.LayerNorm(c["A"].shape[-1], eps=c["eps"]).to(c["A"].dtype)
                S._compute_layernorm_dot_product(layer, c["A"], c["B"], c["n_val"])
            else:
                continue
            assert layer.weight.grad_dot_prod.dtype == c["dot"].dtype, name
            if c.get("bias_dot") is not None:
                assert layer.bias.grad_dot_prod.dtype == c["bias_dot"].dtype, name
            checked += 1
    assert checked == 24
