"""GPU parity at the stated size of every BASELINE configuration, through the reference API
and the C ABI, against the oracle's closed forms.

  configs[0]  MLP 512-1024-1024-10, fp32, 64 train + 16 val rows, 10 SGD steps
  configs[1]  Linear microbench A[32, T, 768], G[32, T, 3072], 8 val rows first,
              T in {128, 512, 1024, 2048}, both algorithms
  configs[2]  GPT-2-small, 12 layers, bf16, 16 + 4 rows, T = 1024: every hooked module's
              dots and every .grad of one step
  configs[3]  GradProj on the GPT-2-medium shape, B = 32, T = 1024, k = 16 x 16
  configs[4]  Pythia-1B shape, 8 + 2 rows, T = 2048: every hooked module (embed_out's
              output gradient is 2.06 GB) and every .grad of one step

The expected values are the oracle's float64 closed forms evaluated on the tensors the
samplers received (captured by hooks of this test), on the GPU where the sizes need it
(2-D float64 products only).  Tolerances: bf16 operands 2e-2 normwise, fp32 operands 1e-4
normwise (|x - y| <= tol * max(|y|, rms(y))); routing (which parameter receives which
result) exact.
"""
import copy

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from ghostsuite_amd import GradDotProdEngine, GradProjLoraEngine, _native
from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
from ghostsuite_amd.workloads import (CausalLM, GPT2_MEDIUM, GPT2_SMALL, MLP, PYTHIA_1B,
                                      LMConfig, synthetic_tokens)
from oracle import brute
from oracle import ghost_ref as R
from tests.helpers import BF16_TOL, FP32_TOL, assert_close, assert_close_to_sum, gen, randn

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


@pytest.fixture(autouse=True)
def _reset_options():
    saved = dict(S.options)
    yield
    S.options.clear()
    S.options.update(saved)


def _say(msg):
    print(msg, flush=True)


class HookCapture:
    """Keeps every sampled module's input and output gradient (the A and B its sampler
    receives), by hooks registered after the engine's."""

    def __init__(self, model, types, names=None):
        self.A, self.B, self.handles = {}, {}, []
        for name, m in model.named_modules():
            if type(m) in types and (names is None or name in names):
                self.handles.append(m.register_forward_hook(self._fwd(name)))
                self.handles.append(m.register_full_backward_hook(self._bwd(name)))

    def _fwd(self, name):
        def hook(m, inp, out):
            self.A[name] = inp[0].detach()
        return hook

    def _bwd(self, name):
        def hook(m, gin, gout):
            self.B[name] = gout[0].detach()
        return hook

    def remove(self):
        for h in self.handles:
            h.remove()


def _param_names(model):
    return {id(p): n for n, p in model.named_parameters()}


def _train_rows(x, n_t):
    return x[:n_t].reshape(-1, x.shape[-1])


def _expected_lm(model, cap, n_t, n_v, reduction="mean"):
    """{param name: expected dot} and {param name: expected .grad}, float64 on the device."""
    N = n_t + n_v
    # the train grads average the backprops, N-scaled for a mean loss, over the train rows
    s = (N if reduction == "mean" else 1) / n_t
    names = _param_names(model)
    dots, grads, mags = {}, {}, {}

    def add(name, g):
        # mags: the sum of the contributions' magnitudes (a tied weight gets two)
        grads[name] = grads[name] + g if name in grads else g
        mags[name] = mags[name] + g.abs() if name in mags else g.abs()

    for mname, m in model.named_modules():
        if mname not in cap.A:
            continue
        A, B = cap.A[mname], cap.B[mname]
        wname = names[id(m.weight)]
        if isinstance(m, nn.Linear):
            tied = wname != f"{mname}.weight"
            if not tied:
                sem = "pairwise" if m.use_ghost_computation else "presum"
                dots[wname] = R.linear_dot_valterm_exact(A, B, n_v, sem)
            add(wname, s * torch.mm(_train_rows(B, n_t).double().t(),
                                    _train_rows(A, n_t).double()))
            if m.bias is not None:
                dots[names[id(m.bias)]] = R.bias_dot_exact(B, n_v)
                add(names[id(m.bias)], s * _train_rows(B, n_t).double().sum(0))
        elif isinstance(m, nn.Embedding):
            dots[wname] = R.embedding_dot_exact(A, B, n_v)
            g = torch.zeros(m.weight.shape, dtype=torch.float64, device=B.device)
            g.index_add_(0, A[:n_t].reshape(-1).long(), _train_rows(B, n_t).double())
            add(wname, s * g)
        elif isinstance(m, nn.LayerNorm):
            dw, db = R.layernorm_dot_exact(A, B, n_v, m.eps)
            dots[wname], dots[names[id(m.bias)]] = dw, db
            xh = F.layer_norm(_train_rows(A, n_t).double(), (A.shape[-1],), eps=m.eps)
            add(wname, s * (_train_rows(B, n_t).double() * xh).sum(0))
            add(names[id(m.bias)], s * _train_rows(B, n_t).double().sum(0))
    return dots, grads, mags


def _lm_step(model, X, Y, n_t, n_v, loss_reduction="mean", **options):
    """One GradDotProd step through the engine (the reference's step order); returns the
    per-parameter dots, the .grad values, the logged aggregate and the capture.  With
    loss_reduction='sum' the loss is the token sum (the model's token mean times N T)."""
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=True,
                            loss_reduction=loss_reduction, **options)
    eng.attach(opt)
    cap = HookCapture(model, tuple(S._supported_layers_dotprod))
    eng.attach_train_batch(X[:n_t], Y[:n_t], 0, 0)
    loss = model(X, Y)
    if loss_reduction == "sum":
        loss = loss * X.numel()
    loss.backward()
    torch.cuda.synchronize()
    dots = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()
            if hasattr(p, "grad_dot_prod")}
    eng.prepare_gradients()
    grads = {n: p.grad for n, p in model.named_parameters()
             if p.grad is not None and "dummy_bias" not in n}
    eng.aggregate_and_log()
    total = eng.dot_product_log[-1]["dot_product"]
    cap.remove()
    return eng, dots, grads, total, cap


def _check_lm(model, dots, grads, total, cap, n_t, n_v, reduction="mean", backwards=1):
    """``backwards``: backward passes of the same batch and weights before the gradients were
    read (gradient accumulation): the train gradients add up, the dots are the last pass's."""
    want_dots, want_grads, mags = _expected_lm(model, cap, n_t, n_v, reduction)
    want_grads = {k: backwards * v for k, v in want_grads.items()}
    mags = {k: backwards * v for k, v in mags.items()}
    contributions = {}
    for mname, m in model.named_modules():
        if mname in cap.A:
            pid = _param_names(model)[id(m.weight)]
            contributions[pid] = contributions.get(pid, 0) + 1
    assert sorted(dots) == sorted(want_dots), (sorted(dots), sorted(want_dots))
    for name in sorted(want_dots):
        worst = assert_close(dots[name], want_dots[name], BF16_TOL, f"dot {name}")
        _say(f"  dot {name}: worst {worst:.2e}")
    assert_close(total, sum(want_dots.values()).cpu(), BF16_TOL, "logged aggregate")
    trainable = sorted(n for n, p in model.named_parameters()
                       if p.initially_requires_grad and "dummy_bias" not in n)
    assert sorted(grads) == trainable and sorted(want_grads) == trainable
    for name in trainable:
        if contributions.get(name, 1) > 1:   # a tied weight: Linear + Embedding train grads
            worst = assert_close_to_sum(grads[name], want_grads[name], mags[name], BF16_TOL,
                                  f"grad {name}")
        else:
            worst = assert_close(grads[name], want_grads[name], BF16_TOL, f"grad {name}")
        _say(f"  grad {name}: worst {worst:.2e}")


# ------------------------------------------------------------------ configs[1]
@pytest.mark.parametrize("T", [128, 512, 1024, 2048])
def test_config1_linear_microbench(gpu, T):
    """A[32, T, 768] ~ N(0, 1), G[32, T, 3072] ~ N(0, 1e-3^2), bf16, the first 8 rows val.
    The reference's switch picks pairwise for T <= 1024 and presum at T = 2048; both
    semantics run through both algorithms at every T."""
    n_val, d_in, d_out = 8, 768, 3072
    A = randn((32, T, d_in), 1234, 1.0, BF16).to(gpu)
    G = randn((32, T, d_out), 1235, 1e-3, BF16).to(gpu)
    assert R.should_use_ghost(T, d_in * d_out) == (T <= 1024)
    for sem_name, sem in (("pairwise", _native.SEM_PAIRWISE_SUM),
                          ("presum", _native.SEM_PRESUM)):
        want = R.linear_dot_valterm_exact(A, G, n_val, sem_name, val_start=0)
        for algo in (_native.ALGO_GHOST, _native.ALGO_VALGRAD):
            _say(f"config1 T={T} sem={sem_name} algo={_native.ALGO_NAMES[algo]}")
            dot, _ = _native.ops().linear_dot(A, G, n_val, val_start=0, semantics=sem,
                                              algo=algo)
            torch.cuda.synchronize()
            assert_close(dot, want, BF16_TOL, f"T={T} {sem_name} {algo}")


def test_config1_reference_sequence_t1024(gpu):
    """The reference's own bf16 op sequence of the ghost branch (bf16 Gram products, bf16
    Hadamard product, fp32 sums; 2-D products on the GPU) at the T = 1024 microbench, with
    the reference layout (val last): the default kernels at 2e-2, the ghost kernel in its
    reference-rounding mode at 2e-3."""
    n_val, T = 8, 1024
    A = randn((32, T, 768), 1240, 1.0, BF16).to(gpu)
    G = randn((32, T, 3072), 1241, 1e-3, BF16).to(gpu)
    want, _ = R.linear_dot_ref(A, G, n_val, use_ghost=True, has_bias=False)
    torch.cuda.synchronize()
    for algo in (_native.ALGO_GHOST, _native.ALGO_VALGRAD):
        _say(f"config1 reference sequence algo={_native.ALGO_NAMES[algo]}")
        dot, _ = _native.ops().linear_dot(A, G, n_val, algo=algo)
        torch.cuda.synchronize()
        assert_close(dot, want, BF16_TOL, f"ref sequence {algo}")
    dot, _ = _native.ops().linear_dot(A, G, n_val, algo=_native.ALGO_GHOST,
                                      rounding=_native.ROUND_REF_BF16)
    torch.cuda.synchronize()
    assert_close(dot, want, 2e-3, "ghost reference rounding")


# ------------------------------------------------------------------ configs[2] samplers
def test_config2_reference_sequences_gpt2_shapes(gpu):
    """Every GPT-2-small sampler the step runs, at its full shape (16 train + 4 val rows,
    T = 1024, bf16, reference layout), against the reference's own op sequence rather than
    the float64 forms: the fused dot + train-gradient op on fc / fc_out (the reference's
    ghost branch: bf16 Gram products, bf16 Hadamard product, fp32 sums; 2-D products on the
    GPU) and on qkv / proj (its materialised branch: per-sample gradients and the presummed
    val gradient in bf16, on the CPU), the HF Conv1D form on c_fc (ghost branch) and c_attn
    (materialised; presum in both, all bf16), bias dots alike, the Embedding on wte and wpe
    (bf16 index_add_ table, bf16 gather-product) and LayerNorm weight / bias dots (bf16
    layer_norm), each within the bf16 tolerance, with the distances printed."""
    from ghostsuite_amd import _native as NV
    N, n_val, T = 20, 4, 1024
    n_t = N - n_val
    ops = NV.ops()
    dist = {}

    def check(name, got, want):
        dist[name] = assert_close(got.float().cpu(), want.float().cpu(), BF16_TOL, name)

    for name, d_in, d_out, seed in (("fc", 768, 3072, 300), ("fc_out", 3072, 768, 302),
                                    ("qkv", 768, 2304, 304), ("proj", 768, 768, 306)):
        ghost = R.should_use_ghost(T, d_in * d_out)
        assert ghost == (name in ("fc", "fc_out"))
        A = randn((N, T, d_in), seed, 1.0, BF16)
        G = randn((N, T, d_out), seed + 1, 1e-3, BF16)
        _say(f"config2 reference sequence {name}")
        dot, _, bdot, _ = ops.linear_dot_train_grad(
            A.to(gpu), G.to(gpu), n_val,
            semantics=NV.SEM_PAIRWISE_SUM if ghost else NV.SEM_PRESUM,
            grad_scale=N / n_t, bias=True, bias_grad_scale=N / n_t)
        torch.cuda.synchronize()
        if ghost:
            w, b = R.linear_dot_ref(A.to(gpu), G.to(gpu), n_val, use_ghost=True)
        else:
            w, b = R.linear_dot_ref(A, G, n_val, use_ghost=False)
        check(f"{name} weight", dot, w)
        check(f"{name} bias", bdot, b)
    for name, d_in, d_out, seed in (("c_fc", 768, 3072, 310), ("c_attn", 768, 2304, 312)):
        A = randn((N, T, d_in), seed, 1.0, BF16)
        G = randn((N, T, d_out), seed + 1, 1e-3, BF16)
        _say(f"config2 reference sequence Conv1D {name}")
        dot, _, bdot, _ = ops.linear_dot_train_grad(
            A.to(gpu), G.to(gpu), n_val, semantics=NV.SEM_PRESUM, grad_scale=N / n_t,
            bias=True, bias_grad_scale=N / n_t, conv1d=True)
        torch.cuda.synchronize()
        w, b = R.conv1d_dot_ref(A, G, n_val, R.should_use_ghost(T, d_in * d_out))
        check(f"{name} weight", dot, w)
        check(f"{name} bias", bdot, b)
    G = randn((N, T, 768), 320, 1e-3, BF16)
    for name, ids, vocab in (("wte", torch.randint(0, 50257, (N, T), generator=gen(321)), 50257),
                             ("wpe", torch.arange(T).repeat(N, 1), T)):
        _say(f"config2 reference sequence embedding {name}")
        dot = ops.embedding_dot(ids.to(gpu), G.to(gpu), n_val, vocab)
        torch.cuda.synchronize()
        check(name, dot, R.embedding_dot_ref(ids, G, n_val, vocab))
    X = randn((N, T, 768), 322, 1.0, BF16)
    _say("config2 reference sequence layernorm")
    dw, db, _, _ = ops.layernorm_dot(X.to(gpu), G.to(gpu), n_val, 1e-5)
    torch.cuda.synchronize()
    w, b = R.layernorm_dot_ref(X, G, n_val, 1e-5)
    check("layernorm weight", dw, w)
    check("layernorm bias", db, b)
    print("normwise distances to the reference sequence: " +
          ", ".join(f"{k} {v:.2e}" for k, v in dist.items()), flush=True)


# ------------------------------------------------------------------ configs[0]
@pytest.mark.parametrize("precision,tol", [("fp32", FP32_TOL), ("reference", BF16_TOL)])
def test_config0_mlp_ten_steps(gpu, precision, tol):
    """Linear 512 -> 1024 -> ReLU -> 1024 -> ReLU -> 10, fp32, 64 train + 16 val rows,
    x ~ N(0, 1), labels uniform over 10 classes, mean cross-entropy, SGD lr 0.1, 10 steps:
    every layer's dots per step and the weights after every step against per-sample
    gradients of a float64 copy (one backward per sample)."""
    torch.manual_seed(0)
    model = MLP((512, 1024, 1024, 10))
    ref = copy.deepcopy(model).double()
    model = model.to(gpu)
    n_t, n_v = 64, 16
    N = n_t + n_v
    X = torch.randn(N, 512, generator=gen(1))
    Y = torch.randint(0, 10, (N,), generator=gen(2))
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=False,
                            precision=precision)
    eng.attach(opt)
    Xd, Yd = X.to(gpu), Y.to(gpu)
    for step in range(10):
        _say(f"config0 precision={precision} step {step}")
        eng.attach_train_batch(Xd[:n_t], Yd[:n_t], step, 0)
        opt.zero_grad(set_to_none=True)
        F.cross_entropy(model(Xd), Yd).backward()
        torch.cuda.synchronize()
        dots = {n: p.grad_dot_prod.cpu() for n, p in model.named_parameters()}
        eng.prepare_gradients()
        opt.step()
        eng.aggregate_and_log()
        eng.clear_gradients()
        g = brute.per_sample_grads(
            ref, X.double(), Y, lambda m, x, y: F.cross_entropy(m(x), y, reduction="sum"),
            1.0 / N)
        for name, gr in g.items():
            # T = 1: every layer takes the ghost branch (pairwise sums); bias dots are in
            # the model dtype in both precisions
            t = tol if name.endswith("weight") else FP32_TOL
            assert_close(dots[name], brute.pairwise_dots(gr, n_v), t, f"step {step} {name}")
        assert_close(eng.dot_product_log[-1]["dot_product"],
                     sum(brute.pairwise_dots(gr, n_v) for gr in g.values()), tol,
                     f"step {step} aggregate")
        with torch.no_grad():
            for name, p in ref.named_parameters():
                p -= 0.1 * brute.train_mean(g[name], n_v, N)
        for (n1, p1), (_, p2) in zip(model.named_parameters(), ref.named_parameters()):
            assert_close(p1.detach().cpu(), p2.detach(), 1e-4, f"step {step} weights {n1}")
    eng.detach()


# ------------------------------------------------------------------ configs[2]
def test_config2_gpt2_small_full_step(gpu):
    """GPT-2-small (12 layers, d = 768, vocab 50257, tied lm_head), N(0, 0.02) weights,
    bf16, 16 train + 4 val rows of uniform token ids, T = 1024, next-token cross-entropy:
    all 76 hooked modules' dots (the tied lm_head's is overwritten by wte's, as in the
    reference) and every .grad after one step."""
    torch.manual_seed(0)
    n_t, n_v, T = 16, 4, 1024
    with torch.device(gpu):
        model = CausalLM(GPT2_SMALL).to(BF16)
    X, Y = synthetic_tokens(n_t + n_v, T, GPT2_SMALL.vocab, seed=5, device=gpu)
    _say("config2 step")
    eng, dots, grads, total, cap = _lm_step(model, X, Y, n_t, n_v)
    hooked = sum(1 for m in model.modules() if type(m) in S._supported_layers_dotprod)
    assert hooked == 76 and len(cap.A) == 76
    sem = {n: m.use_ghost_computation for n, m in model.named_modules()
           if hasattr(m, "use_ghost_computation")}
    assert sem["h.0.fc"] and sem["h.0.fc_out"] and not sem["h.0.qkv"] and not sem["h.0.proj"]
    _check_lm(model, dots, grads, total, cap, n_t, n_v)
    eng.detach()


# ------------------------------------------------------------------ configs[4]
def test_config4_pythia_full_step(gpu):
    """Pythia-1B shape (16 layers, d = 2048, MLP 8192, rotary, untied embed_out over
    vocab 50304), bf16, 8 train + 2 val rows, T = 2048: every hooked module's dots and every
    .grad after one step.  embed_out's output gradient [10, 2048, 50304] bf16 is 2.06 GB."""
    torch.manual_seed(0)
    n_t, n_v, T = 8, 2, 2048
    with torch.device(gpu):
        model = CausalLM(PYTHIA_1B).to(BF16)
    X, Y = synthetic_tokens(n_t + n_v, T, PYTHIA_1B.vocab, seed=9, device=gpu)
    _say("config4 step")
    eng, dots, grads, total, cap = _lm_step(model, X, Y, n_t, n_v)
    assert cap.B["lm_head"].numel() * 2 > 2 * 10 ** 9
    sem = {n: m.use_ghost_computation for n, m in model.named_modules()
           if hasattr(m, "use_ghost_computation")}
    assert sem["h.0.qkv"] and not sem["h.0.proj"] and sem["h.0.fc"] and sem["lm_head"]
    _check_lm(model, dots, grads, total, cap, n_t, n_v)
    eng.detach()


# ------------------------------------------------------------------ configs[3]
def test_config3_gradproj_gpt2_medium(gpu, tmp_path):
    """GPT-2-medium shape (24 layers, d = 1024, MLP 4096), bf16, B = 32, T = 1024, a
    16 x 16 Kronecker projection on each of the 96 block Linear layers (seed 42, fp16
    output): each layer's projection against the float64 projection-first closed form
    (with the bf16 projections the kernels use), and the concatenation in sorted layer-name
    order."""
    torch.manual_seed(0)
    B, T = 32, 1024
    with torch.device(gpu):
        model = CausalLM(GPT2_MEDIUM).to(BF16)
    X, Y = synthetic_tokens(B, T, GPT2_MEDIUM.vocab, seed=77, device=gpu)
    eng = GradProjLoraEngine(model, proj_layers="h.", proj_rank_total=256, proj_rank_min=8,
                             proj_seed=42, proj_dtype="float16", proj_dir=str(tmp_path),
                             proj_dims_override=(16, 16))
    assert len(eng.matched_layers) == 96
    eng.attach()
    cap = HookCapture(model, (nn.Linear,), names=set(eng.matched_layers))
    _say("config3 step")
    model(X, Y).backward()
    torch.cuda.synchronize()
    per_layer = {n: l._ghost_grad_proj.clone() for n, l in eng.matched_layers.items()}
    full = eng.collect_batch()
    torch.cuda.synchronize()
    cap.remove()
    wants = {}
    for name in sorted(eng.matched_layers):
        _say(f"  proj {name}")
        P_i, P_o = eng.projection_matrices[name]
        want = R.kron_proj_projfirst_exact(cap.A[name], cap.B[name], P_i.to(BF16),
                                           P_o.to(BF16), float(B))
        assert_close(per_layer[name], want, BF16_TOL, f"proj {name}")
        wants[name] = want.reshape(B, -1)
    assert_close(full.double(), torch.cat([wants[n] for n in sorted(wants)], dim=1), BF16_TOL,
                 "collected batch")
    assert full.dtype == torch.float16 and full.shape == (B, 96 * 256)
    eng.detach()


def test_config3_gradproj_reference_ranks(gpu, tmp_path):
    """The same model and batch with the projection sizes the reference's choose_ki_ko picks
    at its documented --proj_rank_total 512, k_min 8 (Examples/GradProj_LM/README.md:67),
    embeddings included: (39, 13) qkv, (23, 22) proj, (43, 12) fc, (11, 47) fc_out, (8, 64)
    wte, (23, 22) wpe; every layer against the float64 projection-first closed forms."""
    torch.manual_seed(0)
    B, T = 32, 1024
    with torch.device(gpu):
        model = CausalLM(GPT2_MEDIUM).to(BF16)
    X, Y = synthetic_tokens(B, T, GPT2_MEDIUM.vocab, seed=78, device=gpu)
    eng = GradProjLoraEngine(model, proj_layers="h.,wte,wpe", proj_rank_total=512,
                             proj_rank_min=8, proj_seed=42, proj_dtype="float16",
                             proj_dir=str(tmp_path), include_embeddings=True)
    dims = eng.projection_dims
    assert dims["h.0.qkv"] == (39, 13) and dims["h.0.fc"] == (43, 12)
    assert dims["h.0.fc_out"] == (11, 47) and dims["wte"] == (8, 64)
    eng.attach()
    cap = HookCapture(model, (nn.Linear, nn.Embedding), names=set(eng.matched_layers))
    _say("config3 reference ranks step")
    model(X, Y).backward()
    torch.cuda.synchronize()
    per_layer = {n: l._ghost_grad_proj.clone() for n, l in eng.matched_layers.items()}
    full = eng.collect_batch()
    torch.cuda.synchronize()
    cap.remove()
    wants = {}
    for name in sorted(eng.matched_layers):
        P_i, P_o = eng.projection_matrices[name]
        if isinstance(eng.matched_layers[name], nn.Embedding):
            want = R.kron_embed_proj_projfirst_exact(cap.A[name], cap.B[name], P_i.to(BF16),
                                                     P_o.to(BF16))
        else:
            want = R.kron_proj_projfirst_exact(cap.A[name], cap.B[name], P_i.to(BF16),
                                               P_o.to(BF16), float(B))
        worst = assert_close(per_layer[name], want, BF16_TOL, f"proj {name}")
        _say(f"  proj {name} {tuple(per_layer[name].shape[1:])}: worst {worst:.2e}")
        wants[name] = want.reshape(B, -1)
    assert_close(full.double(), torch.cat([wants[n] for n in sorted(wants)], dim=1), BF16_TOL,
                 "collected batch")
    eng.detach()


# ------------------------------------------------------------------ operands above 2 GiB
def test_linear_operand_above_2gib(gpu):
    """An output gradient of 2.47 GB (12 x 2048 x 50304 bf16), past the 2^31-byte reach of
    the buffer-resource loads: the val-gradient and bias passes take their other kernels;
    dots against the float64 closed forms."""
    N, n_val, T, d_in, d_out = 12, 2, 2048, 256, 50304
    A = randn((N, T, d_in), 71, 1.0, BF16).to(gpu)
    G = randn((N, T, d_out), 72, 1e-3, BF16).to(gpu)
    assert G.numel() * 2 > 2 ** 31
    want = R.linear_dot_valterm_exact(A, G, n_val, "pairwise")
    _say("above-2GiB linear_dot")
    dot, _ = _native.ops().linear_dot(A, G, n_val, algo=_native.ALGO_VALGRAD)
    torch.cuda.synchronize()
    assert_close(dot, want, BF16_TOL, "linear_dot > 2 GiB")
    _say("above-2GiB linear_bias_dot")
    out = _native.ops().linear_bias_dot(A, G, n_val, grad_scale=1.0)
    if out is not None:
        torch.cuda.synchronize()
        assert_close(out[0], want, BF16_TOL, "fused dot > 2 GiB")
        assert_close(out[1], R.bias_dot_exact(G, n_val), BF16_TOL, "fused bias > 2 GiB")
    bdot, _ = _native.ops().bias_dot(G, n_val)
    torch.cuda.synchronize()
    assert_close(bdot, R.bias_dot_exact(G, n_val), BF16_TOL, "bias_dot > 2 GiB")


def test_sum_reduction_lm_step(gpu):
    """loss_reduction='sum' through the fused dot + train-gradient pass (bf16, T = 64, every
    Linear on the val-gradient algorithm): the backprops are not rescaled (the reference
    scales them by N only for 'mean', autograd_grad_sample_dotprod.py:132-134), so the dots
    are those of the token-summed loss and every train gradient -- bias included, whose stage
    divides by n_train either way (:67, :199-222) -- is the train rows' mean; checked against
    the float64 forms on the captured activations and backprops."""
    torch.manual_seed(31)
    T, vocab, n_t, n_v = 64, 64, 3, 2
    cfg = LMConfig(n_layer=1, n_head=2, d_model=64, d_mlp=128, vocab=vocab, n_ctx=T)
    model = CausalLM(cfg).to(gpu, torch.bfloat16)
    X, Y = synthetic_tokens(n_t + n_v, T, vocab, seed=32, device=gpu)
    _say("sum-reduction LM step")
    S.ALGO_LOG.clear()
    eng, dots, grads, total, cap = _lm_step(model, X, Y, n_t, n_v, loss_reduction="sum",
                                            record_algorithms=True, linear_algo="valgrad")
    fused = sorted(k for k, v in S.ALGO_LOG.items() if v[1] == "valgrad+train_grad")
    assert fused == ["h.0.fc", "h.0.fc_out", "h.0.proj", "h.0.qkv"], S.ALGO_LOG
    _check_lm(model, dots, grads, total, cap, n_t, n_v, reduction="sum")
    eng.detach()


def test_gradient_accumulation_lm_steps(gpu):
    """Two backward passes per optimizer step, each on loss / 2 (the reference loop's
    gradient accumulation, Examples/GradDotProd_LM/training_loop.py:122-144), through the
    fused pass (bf16, T = 64): every parameter's dot is the last pass's (the samplers assign
    it), every train gradient the sum of both passes' (added into param.train_grad,
    supported_layers_grad_samplers_dotprod.py:44-70), tied weight included."""
    torch.manual_seed(33)
    T, vocab, n_t, n_v = 64, 64, 3, 2
    cfg = LMConfig(n_layer=1, n_head=2, d_model=64, d_mlp=128, vocab=vocab, n_ctx=T)
    model = CausalLM(cfg).to(gpu, torch.bfloat16)
    X, Y = synthetic_tokens(n_t + n_v, T, vocab, seed=34, device=gpu)
    _say("gradient accumulation, 2 backward passes")
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=True,
                            record_algorithms=True, linear_algo="valgrad")
    eng.attach(opt)
    cap = HookCapture(model, tuple(S._supported_layers_dotprod))
    eng.attach_train_batch(X[:n_t], Y[:n_t], 0, 0)
    S.ALGO_LOG.clear()
    for _ in range(2):
        (model(X, Y) / 2).backward()
    torch.cuda.synchronize()
    fused = sorted(k for k, v in S.ALGO_LOG.items() if v[1] == "valgrad+train_grad")
    assert fused == ["h.0.fc", "h.0.fc_out", "h.0.proj", "h.0.qkv"], S.ALGO_LOG
    dots = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()
            if hasattr(p, "grad_dot_prod")}
    eng.prepare_gradients()
    grads = {n: p.grad for n, p in model.named_parameters()
             if p.grad is not None and "dummy_bias" not in n}
    eng.aggregate_and_log()
    total = eng.dot_product_log[-1]["dot_product"]
    cap.remove()
    _check_lm(model, dots, grads, total, cap, n_t, n_v, backwards=2)
    eng.detach()


def test_autocast_lm_step(gpu):
    """fp32 parameters with a bf16 autocast forward (the reference LM example's setting when
    model_dtype and train_dtype differ, Examples/shared/training_utils.py:193-201): the hooks
    see fp32 and bf16 activations and bf16 output gradients in varying pairs, promoted to a
    common dtype before each dot (autograd_grad_sample_dotprod.py:116-123); the layers whose
    operands are both bf16 take the fused pass.  Every dot and train gradient against the
    float64 forms on the captured operands."""
    torch.manual_seed(35)
    T, vocab, n_t, n_v = 64, 64, 3, 2
    cfg = LMConfig(n_layer=1, n_head=2, d_model=64, d_mlp=128, vocab=vocab, n_ctx=T)
    model = CausalLM(cfg).to(gpu)
    X, Y = synthetic_tokens(n_t + n_v, T, vocab, seed=36, device=gpu)
    _say("autocast LM step")
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=True,
                            record_algorithms=True, linear_algo="valgrad")
    eng.attach(opt)
    cap = HookCapture(model, tuple(S._supported_layers_dotprod))
    eng.attach_train_batch(X[:n_t], Y[:n_t], 0, 0)
    S.ALGO_LOG.clear()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = model(X, Y)
    loss.backward()
    torch.cuda.synchronize()
    kinds = {n: (cap.A[n].dtype, cap.B[n].dtype) for n in cap.A if n.startswith("h.0.")}
    assert len(set(kinds.values())) > 1, kinds   # mixed operand dtypes across the layers
    fused = [n for n, v in S.ALGO_LOG.items() if v[1] == "valgrad+train_grad"]
    assert fused, S.ALGO_LOG   # bf16 operands with fp32 parameters take the fused pass
    dots = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()
            if hasattr(p, "grad_dot_prod")}
    eng.prepare_gradients()
    grads = {n: p.grad for n, p in model.named_parameters()
             if p.grad is not None and "dummy_bias" not in n}
    assert all(g.dtype == torch.float32 for g in grads.values())   # the parameters' dtype
    eng.aggregate_and_log()
    total = eng.dot_product_log[-1]["dot_product"]
    cap.remove()
    _check_lm(model, dots, grads, total, cap, n_t, n_v)
    eng.detach()
