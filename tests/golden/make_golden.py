"""Writes tests/golden/reference_vectors.pt: input/output vectors of the reference's own
functions whose results no closed form, brute-force check or invariant fixes bit for bit.

Run in the build container only (the reference is not present on the GPU box):

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py /root/reference

What is recorded (all on the CPU, small seeded inputs, the reference imported unchanged):
  - the bf16 rounding sequences of the GradDotProd samplers
    (ghostEngines/supported_layers_grad_samplers_dotprod.py): _compute_linear_dot_product in
    both branches (:75-146), _compute_embedding_dot_product (:181-211),
    _compute_layernorm_dot_product (:242-300), _compute_Conv1D_dot_product in both branches
    (:369-471), _compute_conv2d_dot_product's materialised branch (:513-563), each with fp32
    and bf16 inputs;
  - GradDotProdEngine's aggregation and routing with real hook firing order
    (graddotprod_engine.py:131-230, autograd_grad_sample_dotprod.py:23-222) on a small model
    whose output Linear is tied to its input Embedding (the Embedding's later assignment
    overwrites the tied Linear's dot, its train gradient accumulates), over two SGD steps;
  - init_projection_matrix_gaussian's values on the CPU generator
    (gradProjection/projection_utils.py:70-97).

The file holds inputs and outputs only (tensors, ints and strings; load it with
torch.load(..., weights_only=True)).
"""
from __future__ import annotations

import hashlib
import os
import sys

import torch
from torch import nn


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _randn(shape, seed, scale=1.0):
    return torch.randn(shape, generator=_gen(seed)) * scale


def _sampler_vectors(S):
    """{case name: {inputs..., outputs...}} for the dot-product samplers."""
    out = {}
    for dt_name, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        for shape_name, a_shape in (("3d", (6, 5, 12)), ("2d", (6, 12)), ("4d", (6, 2, 3, 12))):
            for ghost in (True, False):
                lin = nn.Linear(12, 20)
                lin.use_ghost_computation = ghost      # the branch, as the switch caches it
                A = _randn(a_shape, 10).to(dt)
                B = _randn(a_shape[:-1] + (20,), 11, 1e-2).to(dt)
                S._compute_linear_dot_product(lin, A, B, 2)
                out[f"linear_{'ghost' if ghost else 'mat'}_{shape_name}_{dt_name}"] = {
                    "A": A, "B": B, "n_val": 2,
                    "dot": lin.weight.grad_dot_prod.detach().clone(),
                    "bias_dot": lin.bias.grad_dot_prod.detach().clone()}
        for vocab in (11, 50):
            emb = nn.Embedding(vocab, 16)
            ids = torch.randint(0, vocab, (6, 7), generator=_gen(12 + vocab))
            B = _randn((6, 7, 16), 13, 1e-2).to(dt)
            S._compute_embedding_dot_product(emb, ids, B, 3)
            out[f"embedding_v{vocab}_{dt_name}"] = {
                "ids": ids, "B": B, "n_val": 3, "vocab": vocab,
                "dot": emb.weight.grad_dot_prod.detach().clone()}
        ln = nn.LayerNorm(24)
        A = (_randn((6, 5, 24), 14, 2.0) + 0.3).to(dt)
        B = _randn((6, 5, 24), 15, 1e-2).to(dt)
        S._compute_layernorm_dot_product(ln, A, B, 2)
        out[f"layernorm_{dt_name}"] = {
            "A": A, "B": B, "n_val": 2, "eps": ln.eps,
            "dot": ln.weight.grad_dot_prod.detach().clone(),
            "bias_dot": ln.bias.grad_dot_prod.detach().clone()}
        try:
            from transformers.pytorch_utils import Conv1D
        except Exception:  # pragma: no cover
            Conv1D = None
        if Conv1D is not None:
            for ghost in (True, False):
                conv = Conv1D(20, 12)   # nf = 20 outputs, nx = 12 inputs
                conv.use_ghost_computation = ghost
                A = _randn((7, 5, 12), 16).to(dt)
                B = _randn((7, 5, 20), 17, 1e-2).to(dt)
                S._compute_Conv1D_dot_product(conv, A, B, 3)
                out[f"conv1d_{'ghost' if ghost else 'mat'}_{dt_name}"] = {
                    "A": A, "B": B, "n_val": 3,
                    "dot": conv.weight.grad_dot_prod.detach().clone(),
                    "bias_dot": conv.bias.grad_dot_prod.detach().clone()}
        # Conv2d, the materialised branch (the ghost branch multiplies [d, d] by [p, p]
        # blocks and needs C_in kh kw == C_out): bf16 unfold, per-sample gradients and the
        # presummed val gradient by einsum, their dot; bias dot alike.
        conv2 = nn.Conv2d(3, 4, kernel_size=3, padding=1, stride=2)
        conv2.use_ghost_computation = False
        A = _randn((6, 3, 8, 8), 18).to(dt)
        B = _randn((6, 4, 4, 4), 19, 1e-2).to(dt)
        S._compute_conv2d_dot_product(conv2, A, B, 2)
        out[f"conv2d_mat_{dt_name}"] = {
            "A": A, "B": B, "n_val": 2, "kernel_size": 3, "padding": 1, "stride": 2,
            "dilation": 1,
            "dot": conv2.weight.grad_dot_prod.detach().clone(),
            "bias_dot": conv2.bias.grad_dot_prod.detach().clone()}
    return out


class TiedNet(nn.Module):
    """Embedding -> LayerNorm -> Linear -> tanh -> output Linear tied to the Embedding."""

    def __init__(self, vocab=13, d=8):
        super().__init__()
        self.emb = nn.Embedding(vocab, d)
        self.ln = nn.LayerNorm(d)
        self.mid = nn.Linear(d, d)
        self.out = nn.Linear(d, vocab, bias=False)
        self.out.weight = self.emb.weight

    def forward(self, x):
        h = self.emb(x)
        h = torch.tanh(self.mid(self.ln(h)))
        return self.out(h)


def tied_net_state(seed=3):
    torch.manual_seed(seed)
    net = TiedNet()
    with torch.no_grad():   # non-trivial LayerNorm affine parameters
        net.ln.weight.copy_(1.0 + 0.1 * torch.randn(8, generator=_gen(seed + 1)))
        net.ln.bias.copy_(0.1 * torch.randn(8, generator=_gen(seed + 2)))
    return net


def tied_net_data():
    X = torch.randint(0, 13, (6, 5), generator=_gen(21))
    Y = torch.randint(0, 13, (6, 5), generator=_gen(22))
    return X, Y


def _engine_vectors(GradDotProdEngine):
    """Two steps of the reference's step order on TiedNet (4 train + 2 val rows, SGD)."""
    net = tied_net_state()
    init = {k: v.detach().clone() for k, v in net.state_dict().items()}
    X, Y = tied_net_data()
    n_t, n_v = 4, 2
    opt = torch.optim.SGD(net.parameters(), lr=0.5)
    eng = GradDotProdEngine(net, val_batch_size=n_v, loss_reduction='mean', use_dummy_bias=False)
    eng.attach(opt)
    steps = []
    for it in range(2):
        eng.attach_train_batch(X[:n_t], Y[:n_t], it, it)
        logits = net(X)
        loss = nn.functional.cross_entropy(logits.reshape(-1, 13), Y.reshape(-1))
        opt.zero_grad()
        loss.backward()
        per_param = {n: p.grad_dot_prod.detach().clone() for n, p in net.named_parameters()
                     if hasattr(p, 'grad_dot_prod')}
        eng.prepare_gradients()
        grads = {n: p.grad.detach().clone() for n, p in net.named_parameters()}
        opt.step()
        eng.aggregate_and_log()
        eng.clear_gradients()
        steps.append({"dots": per_param, "grads": grads,
                      "logged": eng.dot_product_log[-1]['dot_product'].detach().clone()})
    final = {k: v.detach().clone() for k, v in net.state_dict().items()}
    eng.detach()
    return {"init": init, "X": X, "Y": Y, "n_val": n_v, "lr": 0.5, "steps": steps,
            "final": final}


def _projection_vectors(init_fn):
    return {f"gauss_{r}x{c}_s{s}": {"rows": r, "cols": c, "seed": s,
                                    "P": init_fn(r, c, dtype=torch.float32, device='cpu',
                                                 seed=s)}
            for r, c, s in ((5, 7, 42), (16, 64, 1042), (3, 10, 0))}


def _hashes(ref_root):
    files = ["ghostEngines/supported_layers_grad_samplers_dotprod.py",
             "ghostEngines/autograd_grad_sample_dotprod.py",
             "ghostEngines/graddotprod_engine.py",
             "ghostEngines/gradProjection/projection_utils.py"]
    return {f: hashlib.sha256(open(os.path.join(ref_root, f), 'rb').read()).hexdigest()
            for f in files}


def main(ref_root):
    sys.dont_write_bytecode = True   # nothing is written under the reference tree
    sys.path.insert(0, ref_root)
    import transformers
    from ghostEngines import supported_layers_grad_samplers_dotprod as S
    from ghostEngines.graddotprod_engine import GradDotProdEngine
    from ghostEngines.gradProjection.projection_utils import init_projection_matrix_gaussian
    torch.set_num_threads(1)
    data = {
        "meta": {"torch": str(torch.__version__), "transformers": str(transformers.__version__),
                 "threads": 1, "sha256": _hashes(ref_root)},
        "samplers": _sampler_vectors(S),
        "engine_tied": _engine_vectors(GradDotProdEngine),
        "projection": _projection_vectors(init_projection_matrix_gaussian),
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.pt")
    torch.save(data, dst)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
