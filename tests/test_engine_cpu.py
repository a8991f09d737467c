"""Host logic of the engines on the CPU, with the kernel layer replaced by the oracle's
closed forms (tests/oracle_backend.py): hook registration, the ghost/materialise switch,
semantics per layer, tied-weight overwrite, train-gradient routing into .grad, the
named_parameters summation order, error paths, save formats, and GradProj set-up."""
import copy
import json
import types

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from ghostsuite_amd import GhostEngineManager, GradDotProdEngine, GradProjLoraEngine, _native
from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
from ghostsuite_amd.workloads import MLP, CausalLM, LMConfig, synthetic_tokens
from oracle import brute
from oracle import ghost_ref as R
from tests.helpers import BF16_TOL, FP32_TOL, assert_close, conv_net, gen, run_conv_engine
from tests.oracle_backend import use_oracle_backend


@pytest.fixture(autouse=True)
def _reset_options():
    saved = dict(S.options)
    yield
    S.options.clear()
    S.options.update(saved)


def _ce_sum(m, x, y):
    return F.cross_entropy(m(x), y, reduction="sum")


# ------------------------------------------------------------------ MLP
@pytest.mark.parametrize("precision,tol", [("fp32", FP32_TOL), ("reference", BF16_TOL)])
def test_mlp_engine_dots_and_grads_match_per_sample_gradients(precision, tol):
    torch.manual_seed(0)
    dims = (64, 48, 32, 10)
    model = MLP(dims)
    ref = copy.deepcopy(model).double()
    n_t, n_v = 24, 8
    X = torch.randn(n_t + n_v, dims[0], generator=gen(1))
    Y = torch.randint(0, 10, (n_t + n_v,), generator=gen(2))
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    ref_opt = torch.optim.SGD(ref.parameters(), lr=0.1)
    with use_oracle_backend():
        eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=False,
                                precision=precision)
        eng.attach(opt)
        for step in range(3):
            eng.attach_train_batch(X[:n_t], Y[:n_t], step, 0)
            loss = F.cross_entropy(model(X), Y)
            opt.zero_grad(set_to_none=True)
            loss.backward()
            per_param = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()}
            eng.aggregate_and_log()
            eng.prepare_gradients()
            grads_now = {n: p.grad.clone() for n, p in model.named_parameters()}
            opt.step()
            eng.clear_gradients()

            g = brute.per_sample_grads(ref, X.double(), Y, _ce_sum, 1.0 / X.shape[0])
            total = 0
            for name, gr in g.items():
                want = brute.pairwise_dots(gr, n_v)
                assert_close(per_param[name], want, tol, f"step {step} {name}")
                assert_close(grads_now[name], brute.train_mean(gr, n_v, X.shape[0]), FP32_TOL,
                             f"step {step} grad {name}")
                total = total + want
            assert_close(eng.dot_product_log[-1]["dot_product"], total, tol, "aggregate")
            # drive the reference copy with the same train gradients
            for (name, p) in ref.named_parameters():
                p.grad = brute.train_mean(g[name], n_v, X.shape[0])
            ref_opt.step()
        eng.detach()
    assert len(eng.dot_product_log) == 3
    assert set(eng.dot_product_log[0]) == {"dot_product", "X_train", "Y_train", "iter_num",
                                           "batch_idx"}


# ------------------------------------------------------------------ small GPT-2
def _tiny_lm(d=16, T=8, vocab=50):
    return LMConfig(n_layer=2, n_head=2, d_model=d, d_mlp=2 * d, vocab=vocab, n_ctx=T)


def _lm_sample_loss(T):
    def f(m, x, y):
        return m(x, y) * T   # token-mean loss of one row, times its T tokens
    return f


def test_gpt2_engine_routing_and_tied_overwrite():
    torch.manual_seed(3)
    T, vocab = 8, 50
    cfg = _tiny_lm(T=T, vocab=vocab)
    model = CausalLM(cfg)
    untied = CausalLM(cfg)
    untied.load_state_dict(model.state_dict())
    untied.lm_head.weight = nn.Parameter(model.wte.weight.detach().clone())  # same values, own param
    tied_ref = copy.deepcopy(model).double()
    untied = untied.double()
    n_t, n_v = 5, 1
    X, Y = synthetic_tokens(n_t + n_v, T, vocab, seed=4)
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    with use_oracle_backend() as ops:
        eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=True,
                                precision="fp32")
        eng.attach(opt)
        names = {n for n, m in model.named_modules() if hasattr(m, "name")}
        assert {"wte", "wpe", "lm_head", "ln_f", "h.0.qkv", "h.1.fc_out", "h.0.ln_1"} <= names
        eng.attach_train_batch(X[:n_t], Y[:n_t], 0, 0)
        loss = model(X, Y)
        loss.backward()
        # the lm_head dot is overwritten by wte's in the reference; it is not computed here
        linear_shapes = [c[1] for c in ops.calls if c[0] == "linear_dot"]
        assert (n_t + n_v, T, cfg.d_model) in linear_shapes
        assert not any(c[2][-1] == vocab for c in ops.calls if c[0] == "linear_dot")
        dots = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()
                if hasattr(p, "grad_dot_prod")}
        eng.prepare_gradients()
        grads = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
        eng.aggregate_and_log()
        eng.detach()

    N = n_t + n_v
    g_untied = brute.per_sample_grads(untied, X, Y, _lm_sample_loss(T), 1.0 / (N * T))
    g_tied = brute.per_sample_grads(tied_ref, X, Y, _lm_sample_loss(T), 1.0 / (N * T))
    assert "lm_head.weight" not in dots
    for name, d in dots.items():
        want = brute.pairwise_dots(g_untied[name], n_v)   # wte: embedding part only
        assert_close(d, want, FP32_TOL, f"dot {name}")
    # dummy biases get autograd's (zero) grad; the engine leaves them alone
    grads = {n: g for n, g in grads.items() if "dummy_bias" not in n}
    for name, gr in grads.items():
        assert_close(gr, brute.train_mean(g_tied[name], n_v, N), FP32_TOL, f"grad {name}")
    total = sum(brute.pairwise_dots(g_untied[n], n_v) for n in dots)
    assert_close(eng.dot_product_log[-1]["dot_product"], total, FP32_TOL, "aggregate")


def test_switch_selects_semantics_per_layer():
    torch.manual_seed(5)
    T = 16
    cfg = LMConfig(n_layer=1, n_head=2, d_model=8, d_mlp=64, vocab=30, n_ctx=T)
    model = CausalLM(cfg)
    X, Y = synthetic_tokens(5, T, 30, seed=6)
    with use_oracle_backend() as ops:
        eng = GradDotProdEngine(model, val_batch_size=2, use_dummy_bias=True)
        eng.attach(torch.optim.SGD(model.parameters(), lr=0.0))
        model(X, Y).backward()
        eng.detach()
    sems = {c[2][-1] if c[1][-1] == 8 else c[1][-1]: c[3] for c in ops.calls
            if c[0] == "linear_dot"}
    # qkv 8x24=192 < 2*16^2 -> presum; fc 8x64=512 -> ghost (pairwise); fc_out 64x8 likewise
    assert model.h[0].qkv.use_ghost_computation is False
    assert model.h[0].fc.use_ghost_computation is True
    assert sems[24] == _native.SEM_PRESUM
    assert sems[64] == _native.SEM_PAIRWISE_SUM


def test_error_paths():
    model = MLP((8, 4, 3))
    with use_oracle_backend():
        eng = GradDotProdEngine(model, val_batch_size=4, use_dummy_bias=False)
        opt = torch.optim.SGD(model.parameters(), lr=0.1)
        eng.attach(opt)
        with pytest.raises(ValueError, match="twice"):
            from ghostsuite_amd import autograd_grad_sample_dotprod as H
            H.add_hooks(model, 4)
        X = torch.randn(4, 8)
        with pytest.raises(ValueError, match="No training samples"):
            F.cross_entropy(model(X), torch.zeros(4, dtype=torch.long)).backward()
        eng.detach()
    # a trainable parameter outside the supported layers has no train_grad
    m2 = nn.Sequential(nn.Linear(4, 4), nn.Conv1d(1, 1, 1))
    with use_oracle_backend():
        e2 = GradDotProdEngine(m2, val_batch_size=1, use_dummy_bias=False)
        e2.attach(torch.optim.SGD(m2.parameters(), lr=0.1))
        out = m2[0](torch.randn(3, 4)).sum()
        out.backward()
        with pytest.raises(ValueError, match="train_grad"):
            e2.prepare_gradients()
    with pytest.raises(TypeError):
        GradDotProdEngine(MLP((4, 2)), val_batch_size=1, not_an_option=True)


def test_manager_flow_and_save_formats(tmp_path):
    torch.manual_seed(7)
    model = MLP((16, 8, 4))
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    Xv, Yv = torch.randn(3, 16), torch.randint(0, 4, (3,))
    cfg = types.SimpleNamespace(method="GradDotProd", result_dir=str(tmp_path), val_batch_size=3,
                                dot_prod_save_interval=2)
    with use_oracle_backend():
        mgr = GhostEngineManager(cfg, model, opt, {"master_process": True}, (Xv, Yv))
        for model_p in model.parameters():   # the manager always uses the dummy-bias trick
            model_p.requires_grad_(True)
        for it in range(1, 5):
            Xt, Yt = torch.randn(5, 16), torch.randint(0, 4, (5,))
            mgr.attach_train_batch(Xt, Yt, it, batch_idx=it)
            Xc, Yc = mgr.prepare_forward_input(Xt, Yt)
            assert torch.equal(Xc[:5], Xt) and torch.equal(Xc[5:], Xv)
            F.cross_entropy(model(Xc), Yc).backward()
            mgr.prepare_gradients()
            opt.step()
            mgr.aggregate_and_log()
            mgr.clear_gradients()
            opt.zero_grad(set_to_none=True)
            if mgr.should_save_metrics(it):
                mgr.save_metrics(it)
        mgr.cleanup()
    d = tmp_path / "grad_dotprods"
    assert (d / "valset.pt").exists()
    vs = torch.load(d / "valset.pt", weights_only=True)
    assert torch.equal(vs["X_val"], Xv)
    log2 = torch.load(d / "dot_prod_log_iter_2.pt", weights_only=True)
    assert [r["iter_num"] for r in log2] == [1, 2] and log2[0]["dot_product"].shape == (5,)
    assert (d / "dot_prod_log_iter_4.pt").exists()
    assert not hasattr(model, "autograd_grad_sample_hooks")


def test_detach_reattach_gives_same_dots():
    torch.manual_seed(8)
    model = MLP((12, 6, 3))
    X = torch.randn(7, 12)
    Y = torch.randint(0, 3, (7,))
    with use_oracle_backend():
        eng = GradDotProdEngine(model, val_batch_size=2, use_dummy_bias=False, precision="fp32")
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        out = []
        for _ in range(2):
            eng.attach(opt)
            eng.attach_train_batch(X[:5], Y[:5], 0)
            F.cross_entropy(model(X), Y).backward()
            eng.aggregate_and_log()
            eng.prepare_gradients()
            eng.clear_gradients()
            out.append(eng.dot_product_log[-1]["dot_product"])
            eng.detach()
            assert not any(hasattr(p, "train_grad") for p in model.parameters())
    assert torch.allclose(out[0], out[1])


# ------------------------------------------------------------------ GradProj
class SimpleMLP(nn.Module):
    def __init__(self, i=10, h=20, o=5):
        super().__init__()
        self.fc1 = nn.Linear(i, h)
        self.relu = nn.ReLU()
        self.fc2 = nn.Linear(h, o)

    def forward(self, x):
        return self.fc2(self.relu(self.fc1(x)))


def test_gradproj_naive_equality_and_files(tmp_path):
    torch.manual_seed(9)
    model = SimpleMLP()
    X, Y = torch.randn(4, 10), torch.randint(0, 5, (4,))
    conf = dict(proj_layers="fc", proj_rank_total=16, proj_rank_min=2, proj_seed=42,
                proj_dtype="float32", proj_dir=str(tmp_path))
    with use_oracle_backend():
        eng = GradProjLoraEngine(model, **conf)
        eng.attach()
        F.cross_entropy(model(X), Y).backward()
        proj = eng.collect_batch(batch_indices=[0, 1, 2, 3])
        eng.detach()
    # naive: per-sample gradient (batch of 1) then P_o W P_i^T, layers in sorted order
    naive = []
    for b in range(4):
        model.zero_grad()
        F.cross_entropy(model(X[b:b + 1]), Y[b:b + 1]).backward()
        parts = []
        for name in sorted(eng.matched_layers):
            P_i, P_o = eng.projection_matrices[name]
            parts.append((P_o @ eng.matched_layers[name].weight.grad @ P_i.t()).reshape(-1))
        naive.append(torch.cat(parts))
    assert torch.allclose(proj, torch.stack(naive), rtol=1e-4, atol=1e-5)
    saved = torch.load(tmp_path / "proj_iter_000000.pt", weights_only=True)
    assert saved["batch_size"] == 4 and saved["batch_idx"] == [0, 1, 2, 3]
    meta = json.loads((tmp_path / "metadata.json").read_text())
    assert meta["total_proj_dim"] == proj.shape[1]
    assert [l["name"] for l in meta["layers"]] == ["fc1", "fc2"]
    assert meta["layers"][1]["slice_start"] == meta["layers"][0]["slice_end"]


def test_gradproj_non_interference(tmp_path):
    torch.manual_seed(10)
    m1 = SimpleMLP()
    m2 = copy.deepcopy(m1)
    X, Y = torch.randn(8, 10), torch.randint(0, 5, (8,))
    o1 = torch.optim.SGD(m1.parameters(), lr=0.01)
    o2 = torch.optim.SGD(m2.parameters(), lr=0.01)
    with use_oracle_backend():
        eng = GradProjLoraEngine(m2, proj_layers="fc", proj_rank_total=16, proj_rank_min=2,
                                 proj_seed=1, proj_dtype="float16", proj_dir=str(tmp_path))
        eng.attach()
        for _ in range(5):
            for m, o in ((m1, o1), (m2, o2)):
                o.zero_grad()
                F.cross_entropy(m(X), Y).backward()
                o.step()
            assert eng.collect_batch().dtype == torch.float16
        eng.detach()
    for p1, p2 in zip(m1.parameters(), m2.parameters()):
        assert torch.allclose(p1, p2, rtol=1e-5, atol=1e-6)


def test_gradproj_choose_ki_ko_matches_known_answers():
    from ghostsuite_amd.gradProjection.projection_utils import choose_ki_ko
    for (n_i, n_o), want in {(1024, 3072): (28, 9), (3072, 1024): (9, 28),
                             (1024, 4096): (32, 8), (4096, 1024): (8, 32),
                             (1024, 1024): (16, 16)}.items():
        assert choose_ki_ko(n_i, n_o, 256, 8) == want
    for n_i, n_o, k, kmin in [(10, 20, 16, 2), (20, 5, 16, 2), (7, 300, 64, 4), (512, 3, 12, 1)]:
        assert choose_ki_ko(n_i, n_o, k, kmin) == R.choose_ki_ko(n_i, n_o, k, kmin)


def test_gradproj_embedding_projection_matches_naive(tmp_path):
    torch.manual_seed(11)
    emb = nn.Embedding(30, 6)
    model = nn.Sequential(emb, nn.Flatten(), nn.Linear(6 * 4, 3))
    X = torch.randint(0, 30, (3, 4))
    Y = torch.randint(0, 3, (3,))
    with use_oracle_backend():
        eng = GradProjLoraEngine(model, proj_layers="0", proj_rank_total=12, proj_rank_min=2,
                                 proj_seed=5, proj_dtype="float32", proj_dir=str(tmp_path),
                                 include_embeddings=True)
        eng.attach()
        F.cross_entropy(model(X), Y).backward()
        got = eng.matched_layers["0"]._ghost_grad_proj.clone()
        eng.detach()
    P_i, P_o = eng.projection_matrices["0"]
    for b in range(3):
        model.zero_grad()
        F.cross_entropy(model(X[b:b + 1]), Y[b:b + 1], reduction="sum").backward()
        W = emb.weight.grad   # [V, d]: per-sample grad of the embedding table
        naive = P_o @ W.t() @ P_i.t()
        # the reference does not multiply embedding projections by the batch size
        assert torch.allclose(got[b] * 3, naive, rtol=1e-4, atol=1e-6)


# ------------------------------------------------------------------ Conv2d
@pytest.mark.parametrize("n_val", [1, 3])
def test_conv2d_engine_dots_and_grads(n_val):
    torch.manual_seed(60)
    model = conv_net()
    ref = copy.deepcopy(model).double()
    N = 7
    X = torch.randn(N, 3, 8, 8, generator=gen(61))
    Y = torch.randint(0, 5, (N,), generator=gen(62))
    with use_oracle_backend() as ops:
        dots, grads = run_conv_engine(model, X, Y, n_val, "cpu")
        assert sum(1 for c in ops.calls if c[0] == "linear_dot") == 3
    g = brute.per_sample_grads(ref, X.double(), Y, _ce_sum, 1.0 / N)
    if n_val == 1:   # presum (Conv2d) and pairwise (Linear) coincide
        for name, d in dots.items():
            assert_close(d, brute.pairwise_dots(g[name], n_val), FP32_TOL, f"dot {name}")
    for name, gr in grads.items():
        assert_close(gr, brute.train_mean(g[name], n_val, N), FP32_TOL, f"grad {name}")
    assert model[0].use_ghost_computation == (2 * 16 ** 2 <= 6 * 3 * 9)


@pytest.mark.parametrize("n_val", [1, 2])
def test_conv2d_reference_ghost_option(n_val):
    """reference_conv2d_ghost: the Conv2d layer on the ghost branch gets the reference's
    ghost-branch quantity; the one on the materialised branch keeps the presum dot; the train
    gradients are unchanged."""
    from tests.helpers import conv_net_square
    torch.manual_seed(63)
    model = conv_net_square()
    ref = copy.deepcopy(model).double()
    N = 6
    X = torch.randn(N, 4, 8, 8, generator=gen(64))
    Y = torch.randint(0, 5, (N,), generator=gen(65))
    caps = {}
    for idx in (0, 2):
        model[idx].register_forward_hook(
            lambda m, i, o, k=idx: caps.__setitem__(("A", k), i[0].detach().clone()))
        model[idx].register_full_backward_hook(
            lambda m, gi, go, k=idx: caps.__setitem__(("B", k), go[0].detach().clone()))
    with use_oracle_backend():
        dots, grads = run_conv_engine(model, X, Y, n_val, "cpu", reference_conv2d_ghost=True)
    assert model[0].use_ghost_computation and not model[2].use_ghost_computation
    convs = {idx: dict(kernel_size=model[idx].kernel_size, dilation=model[idx].dilation,
                       padding=model[idx].padding, stride=model[idx].stride) for idx in (0, 2)}
    assert_close(dots["0.weight"], R.conv2d_ghost_exact(caps[("A", 0)], caps[("B", 0)], n_val,
                                                        convs[0]), FP32_TOL, "ghost branch")
    assert_close(dots["2.weight"], R.conv2d_dot_exact(caps[("A", 2)], caps[("B", 2)], n_val,
                                                      convs[2]), FP32_TOL, "materialised")
    g = brute.per_sample_grads(ref, X.double(), Y, _ce_sum, 1.0 / N)
    for name, gr in grads.items():
        assert_close(gr, brute.train_mean(g[name], n_val, N), FP32_TOL, f"grad {name}")


def test_conv2d_reference_ghost_option_rejects_non_square_blocks():
    """On the ghost branch with C_in*kh*kw != C_out the reference's elementwise product of the
    two Grams fails; the option raises there too."""
    model = torch.nn.Sequential(torch.nn.Conv2d(2, 5, kernel_size=2, stride=2),
                                torch.nn.Flatten(), torch.nn.Linear(5 * 2 * 2, 3))
    X = torch.randn(4, 2, 4, 4, generator=gen(66))   # L = 4: 2 L^2 <= 5 * 8, ghost branch
    Y = torch.randint(0, 3, (4,), generator=gen(67))
    with use_oracle_backend(), pytest.raises(RuntimeError, match="C_in\\*kh\\*kw"):
        run_conv_engine(model, X, Y, 1, "cpu", reference_conv2d_ghost=True)


def test_options_do_not_carry_over_between_engines():
    S = __import__("ghostsuite_amd.supported_layers_grad_samplers_dotprod",
                   fromlist=["options"])
    with use_oracle_backend():
        GradDotProdEngine(MLP((4, 3)), val_batch_size=1, precision="fp32", overlap=False)
        assert S.options["precision"] == "fp32" and S.options["overlap"] is False
        GradDotProdEngine(MLP((4, 3)), val_batch_size=1)
        assert S.options == S.DEFAULT_OPTIONS


def test_each_engine_runs_with_its_own_options():
    """Two engines on two models: each model's backward runs with its engine's options, and a
    direct change to the shared dict stays with the engine that was installed when it was
    made."""
    torch.manual_seed(0)
    m1, m2 = MLP((6, 5, 3)), MLP((6, 5, 3))
    x = torch.randn(4, 6, generator=gen(3))
    y = torch.randint(0, 3, (4,), generator=gen(4))
    seen = []
    orig = S._supported_layers_dotprod[nn.Linear]

    def spy(layer, A, B, val_batch_size):
        seen.append((S.options["precision"], S.options["overlap"]))
        return orig[0](layer, A, B, val_batch_size)

    with use_oracle_backend():
        e1 = GradDotProdEngine(m1, val_batch_size=1, precision="fp32", overlap=False)
        e1.attach(torch.optim.SGD(m1.parameters(), lr=0.0))
        e2 = GradDotProdEngine(m2, val_batch_size=1)
        e2.attach(torch.optim.SGD(m2.parameters(), lr=0.0))
        S._supported_layers_dotprod[nn.Linear] = (spy, orig[1])
        try:
            for m, want in ((m1, ("fp32", False)), (m2, ("reference", True)),
                            (m1, ("fp32", False))):
                seen.clear()
                F.cross_entropy(m(x), y).backward()
                assert seen and all(s == want for s in seen), (want, seen)
            S.options["linear_algo"] = "valgrad"      # a direct change while e1 is installed
            F.cross_entropy(m2(x), y).backward()
            assert S.options["linear_algo"] == "auto" and e1.options["linear_algo"] == "valgrad"
            F.cross_entropy(m1(x), y).backward()
            assert S.options["linear_algo"] == "valgrad" and e2.options["linear_algo"] == "auto"
        finally:
            S._supported_layers_dotprod[nn.Linear] = orig
            e1.detach()
            e2.detach()


@pytest.mark.parametrize("promote", [False, True])
def test_embedding_id_promotion(promote):
    """The reference's hook promotes an Embedding's int64 ids to the backprops' dtype
    (autograd_grad_sample_dotprod.py:116-123); in a bf16 model ids >= 256 round (1023 ->
    1024, 50000 -> 49920) before its sampler casts them back to long.  By default this
    package uses the ids as given; reference_id_promotion=True reproduces the rounding.
    The two values differ on such ids."""
    from oracle import ghost_ref as R
    vocab, d, T = 1100, 8, 6
    emb = nn.Embedding(vocab, d).to(torch.bfloat16)
    ids = torch.tensor([[1023, 300, 5, 700, 1023, 17], [1024, 301, 5, 701, 1022, 18],
                        [1023, 1021, 6, 700, 299, 17]])
    n_v = 1
    with use_oracle_backend():
        eng = GradDotProdEngine(emb, val_batch_size=n_v, use_dummy_bias=False,
                                reference_id_promotion=promote)
        eng.attach(torch.optim.SGD(emb.parameters(), lr=0.0))
        head = torch.randn(3, T, d, generator=gen(70)).to(torch.bfloat16)
        (emb(ids).float() * head.float()).sum().backward()
        got = emb.weight.grad_dot_prod.clone()
        train_grad = emb.weight.train_grad.clone()
        eng.detach()
    B = head.float()
    exact = R.embedding_dot_exact(ids, B, n_v)
    rounded_ids = ids.to(torch.bfloat16).long()
    bucketed = R.embedding_dot_exact(rounded_ids, B, n_v)
    assert not torch.allclose(exact, bucketed)
    assert_close(got, bucketed if promote else exact, 1e-6, "promotion")
    # The train gradient comes from the ids as given in both settings (the reference's
    # gradient stage reads layer.activations): rows 1022 and 1023, whose ids round to 1024,
    # keep their own contributions.
    N, n_t = ids.shape[0], ids.shape[0] - n_v
    want = torch.zeros(vocab, d, dtype=torch.float64)
    want.index_add_(0, ids[:n_t].reshape(-1), head[:n_t].double().reshape(-1, d) * N / n_t)
    assert want[1023].abs().sum() > 0 and want[1022].abs().sum() > 0
    assert_close(train_grad.double(), want, BF16_TOL, "train grad from the unrounded ids")
    assert torch.equal(train_grad[1020:1030].double() != 0, want[1020:1030] != 0)
    # the reference's own op sequence on the promoted ids is the bucketed value
    assert_close(R.embedding_dot_ref(ids.to(torch.bfloat16), B, n_v, vocab), bucketed,
                 BF16_TOL, "reference sequence")


def test_gradient_stage_skips_side_stream_only_when_everything_is_parked():
    """The hook's gradient stage leaves the side stream alone only when the dot stage parked
    every train gradient the layer applies (weight, and the bias when it trains)."""
    from ghostsuite_amd.autograd_grad_sample_dotprod import _train_grads_parked
    lin = nn.Linear(4, 3)
    for p in lin.parameters():
        p.initially_requires_grad = True
    assert not _train_grads_parked(lin)
    lin._gs_weight_train_grad = torch.zeros(3, 4)
    assert not _train_grads_parked(lin)            # bias trains and is not parked
    lin._gs_bias_train_grad = torch.zeros(3)
    assert _train_grads_parked(lin)
    lin.bias.initially_requires_grad = False
    del lin._gs_bias_train_grad
    assert _train_grads_parked(lin)                # a frozen bias needs nothing
    lin.weight.initially_requires_grad = False
    assert not _train_grads_parked(lin)            # nothing parked for a frozen weight
    ln = nn.LayerNorm(4)
    assert not _train_grads_parked(ln)
    ln._gs_ln_train_grads = (torch.zeros(4), torch.zeros(4))
    assert _train_grads_parked(ln)
    emb = nn.Embedding(5, 4)
    emb.weight.initially_requires_grad = True
    assert not _train_grads_parked(emb)
    emb._gs_weight_train_grad = S.APPLIED          # added into a tied weight's train_grad
    assert _train_grads_parked(emb)


def test_dot_dtypes_follow_the_reference():
    """Each grad_dot_prod comes in the dtype the reference's sampler returns for a bf16
    layer: fp32 from a ghost branch (its fp32 sums, supported_layers_grad_samplers_dotprod.py
    :129-130, :437, :550) and from Embedding / LayerNorm, the operands' dtype from a
    materialised branch and from every bias dot (einsums, :131-146, :445-471, :552-559) --
    the dtypes of the oracle's restatement of those sequences.  dot_dtypes='fp32' keeps every
    dot fp32, and the reference-dtype dots are those fp32 values rounded once."""
    from transformers.pytorch_utils import Conv1D
    bf = torch.bfloat16
    N, n_v = 5, 2

    def run():
        got = {}
        for T, ghost in ((3, True), (12, False)):   # 2 T^2 <= 12 x 10 or not
            A = torch.randn(N, T, 12, generator=gen(T)).to(bf)
            B = (torch.randn(N, T, 10, generator=gen(T + 1)) * 1e-2).to(bf)
            lin = nn.Linear(12, 10).to(bf)
            S._compute_linear_dot_product(lin, A, B, n_v)
            assert lin.use_ghost_computation == ghost
            w_ref, b_ref = R.linear_dot_ref(A, B, n_v, ghost)
            got[f"linear {ghost}"] = (lin, w_ref.dtype, b_ref.dtype)
            conv = Conv1D(10, 12).to(bf)
            S._compute_Conv1D_dot_product(conv, A, B, n_v)
            assert conv.use_ghost_computation == ghost
            w_ref, b_ref = R.conv1d_dot_ref(A, B, n_v, ghost)
            got[f"conv1d {ghost}"] = (conv, w_ref.dtype, b_ref.dtype)
        c2 = nn.Conv2d(3, 4, 3, padding=1, stride=2).to(bf)
        X = torch.randn(N, 3, 6, 6, generator=gen(5)).to(bf)
        Gc = (torch.randn(N, 4, 3, 3, generator=gen(6)) * 1e-2).to(bf)
        S._compute_conv2d_dot_product(c2, X, Gc, n_v)
        # the reference's Conv2d casts to bf16 and returns its einsums (:522-559)
        got["conv2d"] = (c2, torch.float32 if c2.use_ghost_computation else bf, bf)
        emb = nn.Embedding(30, 8).to(bf)
        ids = torch.randint(0, 30, (N, 7), generator=gen(7))
        S._compute_embedding_dot_product(emb, ids, (torch.randn(N, 7, 8, generator=gen(8)) *
                                                     1e-2).to(bf), n_v)
        got["embedding"] = (emb, torch.float32, None)
        ln = nn.LayerNorm(8).to(bf)
        S._compute_layernorm_dot_product(ln, torch.randn(N, 7, 8, generator=gen(9)).to(bf),
                                         (torch.randn(N, 7, 8, generator=gen(10)) * 1e-2).to(bf),
                                         n_v)
        got["layernorm"] = (ln, torch.float32, torch.float32)
        return {k: (lay.weight.grad_dot_prod, w, None if b is None else lay.bias.grad_dot_prod, b)
                for k, (lay, w, b) in got.items()}

    with use_oracle_backend():
        S.options["dot_dtypes"] = "fp32"
        full = run()
        S.options["dot_dtypes"] = "reference"
        ref = run()
    assert ref["linear False"][1] == bf and ref["linear True"][1] == torch.float32
    for name, (w, w_dt, b, b_dt) in ref.items():
        fw, _, fb, _ = full[name]
        assert fw.dtype == torch.float32 and w.dtype == w_dt, name
        assert torch.equal(w, fw.to(w_dt)), name
        if b_dt is not None:
            assert fb.dtype == torch.float32 and b.dtype == b_dt, name
            assert torch.equal(b, fb.to(b_dt)), name


def test_sum_reduction_engine_dots_and_grads():
    """loss_reduction='sum': the backprops are not rescaled (the reference scales them by N
    only for 'mean', autograd_grad_sample_dotprod.py:132-134), so the dots are those of the
    summed loss's per-sample gradients and every train gradient -- bias included, whose
    stage divides by n_train either way (:67, :199-222) -- is their mean over the train rows."""
    torch.manual_seed(3)
    dims = (40, 24, 10)
    model = MLP(dims)
    ref = copy.deepcopy(model).double()
    n_t, n_v = 12, 4
    X = torch.randn(n_t + n_v, dims[0], generator=gen(11))
    Y = torch.randint(0, 10, (n_t + n_v,), generator=gen(12))
    with use_oracle_backend():
        eng = GradDotProdEngine(model, val_batch_size=n_v, loss_reduction="sum",
                                use_dummy_bias=False, precision="fp32")
        eng.attach(torch.optim.SGD(model.parameters(), lr=0.0))
        eng.attach_train_batch(X[:n_t], Y[:n_t], 0, 0)
        F.cross_entropy(model(X), Y, reduction="sum").backward()
        dots = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()}
        eng.prepare_gradients()
        grads = {n: p.grad.clone() for n, p in model.named_parameters()}
        eng.clear_gradients()
        eng.detach()
    g = brute.per_sample_grads(ref, X.double(), Y, _ce_sum, 1.0)
    for name, gr in g.items():
        assert_close(dots[name], brute.pairwise_dots(gr, n_v), FP32_TOL, f"dot {name}")
        assert_close(grads[name], brute.train_mean(gr, n_v, 1.0), FP32_TOL, f"grad {name}")


def test_gradient_accumulation_over_backward_passes():
    """Several backward passes before prepare_gradients (the reference loop's gradient
    accumulation, Examples/GradDotProd_LM/training_loop.py:122-144, each on loss / k):
    grad_dot_prod is the last pass's (assigned), train_grad the sum of every pass's (added in
    place, supported_layers_grad_samplers_dotprod.py:44-70)."""
    torch.manual_seed(4)
    dims = (32, 24, 10)
    model = MLP(dims)
    ref = copy.deepcopy(model).double()
    n_t, n_v, k = 10, 3, 3
    X = torch.randn(n_t + n_v, dims[0], generator=gen(21))
    Y = torch.randint(0, 10, (n_t + n_v,), generator=gen(22))
    with use_oracle_backend():
        eng = GradDotProdEngine(model, val_batch_size=n_v, use_dummy_bias=False,
                                precision="fp32")
        eng.attach(torch.optim.SGD(model.parameters(), lr=0.0))
        eng.attach_train_batch(X[:n_t], Y[:n_t], 0, 0)
        for _ in range(k):
            (F.cross_entropy(model(X), Y) / k).backward()
        dots = {n: p.grad_dot_prod.clone() for n, p in model.named_parameters()}
        eng.prepare_gradients()
        grads = {n: p.grad.clone() for n, p in model.named_parameters()}
        eng.clear_gradients()
        eng.detach()
    N = n_t + n_v
    g = brute.per_sample_grads(ref, X.double(), Y, _ce_sum, 1.0 / (N * k))
    for name, gr in g.items():
        assert_close(dots[name], brute.pairwise_dots(gr, n_v), FP32_TOL, f"dot {name}")
        assert_close(grads[name], k * brute.train_mean(gr, n_v, N), FP32_TOL, f"grad {name}")
