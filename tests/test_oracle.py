"""Pins the oracle (oracle/ghost_ref.py) independently of its own formulas: brute-force
per-sample gradients (one backward per sample), invariants, and known answers read off the
reference source.  CPU only."""
import math

import pytest
import torch
from torch import nn

from oracle import brute
from oracle import ghost_ref as R
from tests.helpers import BF16_TOL, assert_close, gen, randn

torch.set_default_dtype(torch.float32)


class Capture:
    """Records a module's input and the grad of the loss w.r.t. its output."""

    def __init__(self, module):
        self.A = self.B = None
        module.register_forward_hook(self._fwd)
        module.register_full_backward_hook(self._bwd)

    def _fwd(self, m, inp, out):
        self.A = inp[0].detach()

    def _bwd(self, m, gin, gout):
        self.B = gout[0].detach()


def _head(seed, d_out):
    return randn((d_out,), seed)


def _run_layer(layer, X, head, N):
    """Mean-over-rows loss sum_t tanh(layer(x)) . head / N; returns (A, B) of the layer."""
    cap = Capture(layer)
    layer.zero_grad()
    out = layer(X)
    loss = (torch.tanh(out) * head).reshape(N, -1).sum(1).mean()
    loss.backward()
    return cap.A, cap.B


def _sample_loss(head):
    return lambda m, x, y: (torch.tanh(m(x)) * head).sum()


# ------------------------------------------------------------------ Linear
@pytest.mark.parametrize("shape", [(7, 2, 3, 5, 4), (6, 1, 4, 3, 6), (5, 3, 1, 8, 2)])
def test_linear_closed_forms_match_per_sample_gradients(shape):
    N, n_val, T, d_in, d_out = shape
    lin = nn.Linear(d_in, d_out).double()
    X = randn((N, T, d_in), 1).double()
    head = _head(2, d_out).double()
    A, B = _run_layer(lin, X, head, N)
    grads = brute.per_sample_grads(lin, X, X, _sample_loss(head), 1.0 / N)
    gw, gb = grads["weight"], grads["bias"]
    # pairwise-sum (ghost branch) == <g_i, sum_j g_j>
    assert_close(R.linear_dot_exact(A, B, n_val, "pairwise"), brute.pairwise_dots(gw, n_val),
                 1e-10, "pairwise")
    assert_close(R.linear_dot_exact(A, B, n_val, "pairwise", pair=True),
                 brute.pair_matrix(gw, n_val), 1e-10, "pair")
    assert_close(R.bias_dot_exact(B, n_val), brute.pairwise_dots(gb, n_val), 1e-10, "bias")
    # the pairwise val term is the summed per-sample val gradient
    assert_close(R.val_term_exact(A, B, n_val, "pairwise"), gw[N - n_val:].sum(0), 1e-10,
                 "val term")
    # train gradient: sum over train rows of (N * g_i) / n_train
    assert_close(R.linear_train_grad(A, B * N, n_val), brute.train_mean(gw, n_val, N), 1e-10,
                 "train grad")
    assert_close(R.bias_train_grad(B * N, n_val), brute.train_mean(gb, n_val, N), 1e-10,
                 "bias train grad")


def test_presum_by_explicit_token_loops():
    N, n_val, T, d_in, d_out = 5, 2, 3, 4, 3
    A = randn((N, T, d_in), 3).double()
    B = randn((N, T, d_out), 4).double()
    n_t = N - n_val
    abar = A[n_t:].sum(0)
    bbar = B[n_t:].sum(0)
    want = torch.zeros(n_t, dtype=torch.float64)
    for i in range(n_t):
        for t in range(T):
            for s in range(T):
                want[i] += (A[i, t] @ abar[s]) * (B[i, t] @ bbar[s])
    assert_close(R.linear_dot_exact(A, B, n_val, "presum"), want, 1e-12, "presum loops")
    V = torch.zeros(d_out, d_in, dtype=torch.float64)
    for t in range(T):
        V += torch.outer(bbar[t], abar[t])
    assert_close(R.val_term_exact(A, B, n_val, "presum"), V, 1e-12, "presum val term")
    # presum == pairwise when there is one val row
    assert_close(R.linear_dot_exact(A[:4], B[:4], 1, "presum"),
                 R.linear_dot_exact(A[:4], B[:4], 1, "pairwise"), 1e-12, "n_val=1")


def test_linear_homogeneity_and_val_layouts():
    N, n_val, T, d_in, d_out = 6, 2, 4, 5, 3
    A = randn((N, T, d_in), 5).double()
    B = randn((N, T, d_out), 6).double()
    base = R.linear_dot_exact(A, B, n_val)
    assert_close(R.linear_dot_exact(2.0 * A, 3.0 * B, n_val), base * 36.0, 1e-12, "homog")
    # the val block moved to the front gives the same numbers for the same rows
    perm = torch.cat([torch.arange(N - n_val, N), torch.arange(0, N - n_val)])
    assert_close(R.linear_dot_exact(A[perm], B[perm], n_val, val_start=0), base, 1e-12, "layout")


@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
@pytest.mark.parametrize("val_start", [None, 0, 2])
def test_linear_val_term_form_equals_closed_form(semantics, val_start):
    """The full-size form (train rows against the val term, one row at a time) against the
    per-sample-gradient closed form; a transposed val term (V^T in place of V, only
    possible with d_in == d_out) is rejected."""
    N, n_val, T, d_in, d_out = 7, 3, 5, 6, 4
    A = randn((N, T, d_in), 51).double()
    B = randn((N, T, d_out), 52).double()
    want = R.linear_dot_exact(A, B, n_val, semantics, val_start=val_start)
    assert_close(R.linear_dot_valterm_exact(A, B, n_val, semantics, val_start=val_start), want,
                 1e-12, "val-term form")
    Asq = randn((N, T, 4), 53).double()
    V = R.val_term_exact(Asq, B, n_val, semantics)
    wrong = torch.stack([(B[i] @ V.t() * Asq[i]).sum() for i in range(N - n_val)])
    ok, _ = R.normwise_close(wrong, R.linear_dot_valterm_exact(Asq, B, n_val, semantics), 1e-3)
    assert not ok


@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
def test_linear_val_term_rounding_points(semantics):
    """The val-term form with the kernels' bf16 rounding points (presummed val rows and V):
    on small-integer inputs every presummed row and every V entry is exactly representable
    in bf16, so the rounded form equals the exact one bit for bit (no term dropped, nothing
    transposed); on random inputs the rounding moves V, and only V, by bf16 relative error,
    and the rounded form equals the dot against that rounded V."""
    N, n_val, T, d_in, d_out = 7, 3, 5, 6, 4
    g = torch.Generator().manual_seed(54)
    Ai = torch.randint(-2, 3, (N, T, d_in), generator=g).double()
    Bi = torch.randint(-2, 3, (N, T, d_out), generator=g).double()
    exact = R.linear_dot_valterm_exact(Ai, Bi, n_val, semantics)
    assert torch.equal(R.linear_dot_valterm_exact(Ai, Bi, n_val, semantics,
                                                  round_dtype=torch.bfloat16), exact)
    A = randn((N, T, d_in), 55).bfloat16()
    B = randn((N, T, d_out), 56, 1e-3).bfloat16()
    V = R.val_term_exact(A, B, n_val, semantics)          # [d_out, d_in], float64
    if semantics == "presum":
        vs = N - n_val
        V = B[vs:].double().sum(0).bfloat16().double().t() @ \
            A[vs:].double().sum(0).bfloat16().double()
    Vr = V.bfloat16().double()
    assert 0 < (Vr - V).abs().max() <= 2.0 ** -8 * V.abs().max()
    want = torch.stack([(B[i].double() @ Vr * A[i].double()).sum() for i in range(N - n_val)])
    assert_close(R.linear_dot_valterm_exact(A, B, n_val, semantics, round_dtype=torch.bfloat16),
                 want, 1e-12, "rounded val-term form")


@pytest.mark.parametrize("T", [1, 6])
def test_linear_reference_sequence_within_bf16_tolerance(T):
    N, n_val, d_in, d_out = 8, 2, 32, 24
    A = randn((N, T, d_in), 7)
    B = randn((N, T, d_out), 8, 1e-3)
    w, b = R.linear_dot_ref(A, B, n_val, use_ghost=True)
    assert_close(w, R.linear_dot_exact(A, B, n_val, "pairwise"), BF16_TOL, "ghost ref")
    assert_close(b, R.bias_dot_exact(B, n_val), 1e-5, "bias ref")
    w2, _ = R.linear_dot_ref(A, B, n_val, use_ghost=False)
    assert_close(w2, R.linear_dot_exact(A, B, n_val, "presum"), 1e-5, "materialised ref")
    pair = R.linear_pair_ref(A, B, n_val)
    assert_close(pair.sum(0), w, 1e-5, "pair sums")
    assert_close(pair, R.linear_dot_exact(A, B, n_val, pair=True), BF16_TOL, "pair ref")


# ------------------------------------------------------------------ Embedding
@pytest.mark.parametrize("V", [5, 40])
def test_embedding_forms_match_per_sample_gradients(V):
    N, n_val, T, d = 7, 3, 6, 4
    emb = nn.Embedding(V, d).double()
    ids = torch.randint(0, V, (N, T), generator=gen(9))
    head = _head(10, d).double()
    A, B = _run_layer(emb, ids, head, N)
    grads = brute.per_sample_grads(emb, ids, ids, _sample_loss(head), 1.0 / N)["weight"]
    want = brute.pairwise_dots(grads, n_val)
    assert_close(R.embedding_dot_exact(A, B, n_val), want, 1e-10, "mask x gram")
    assert_close(R.embedding_dot_ref(A, B.float(), n_val, V), want, BF16_TOL, "ref seq")
    gtr = R.embedding_train_grad(A, B * N, n_val, emb.weight.shape)
    assert_close(gtr, brute.train_mean(grads, n_val, N), 1e-10, "train grad")


# ------------------------------------------------------------------ LayerNorm
def test_layernorm_forms_match_per_sample_gradients():
    N, n_val, T, Fd = 6, 2, 5, 8
    ln = nn.LayerNorm(Fd).double()
    with torch.no_grad():
        ln.weight.copy_(randn((Fd,), 11).double())
        ln.bias.copy_(randn((Fd,), 12).double())
    X = randn((N, T, Fd), 13, 2.0).double() + 0.3
    head = _head(14, Fd).double()
    A, B = _run_layer(ln, X, head, N)
    grads = brute.per_sample_grads(ln, X, X, _sample_loss(head), 1.0 / N)
    ww, wb = R.layernorm_dot_exact(A, B, n_val, ln.eps)
    assert_close(ww, brute.pairwise_dots(grads["weight"], n_val), 1e-10, "ln w")
    assert_close(wb, brute.pairwise_dots(grads["bias"], n_val), 1e-10, "ln b")
    rw, rb = R.layernorm_dot_ref(A.float(), B.float(), n_val, ln.eps)
    assert_close(rw, ww, BF16_TOL, "ln ref w")
    assert_close(rb, wb, BF16_TOL, "ln ref b")
    gw, gb = R.layernorm_train_grad(A, B * N, n_val, ln.eps)
    assert_close(gw, brute.train_mean(grads["weight"], n_val, N), 1e-10, "ln gw")
    assert_close(gb, brute.train_mean(grads["bias"], n_val, N), 1e-10, "ln gb")


# ------------------------------------------------------------------ HF Conv1D
def test_conv1d_reference_is_presum():
    transformers = pytest.importorskip("transformers")
    N, n_val, T, nx, nf = 6, 2, 5, 8, 12
    A = randn((N, T, nx), 15)
    B = randn((N, T, nf), 16, 1e-2)
    want = R.linear_dot_exact(A, B, n_val, "presum")
    for ghost in (True, False):
        w, b = R.conv1d_dot_ref(A, B, n_val, ghost)
        assert_close(w, want, BF16_TOL, f"conv1d ghost={ghost}")
        assert_close(b, R.bias_dot_exact(B, n_val), BF16_TOL, "conv1d bias")


# ------------------------------------------------------------------ GradProj
@pytest.mark.parametrize("conv1d", [False, True])
def test_kron_projection_matches_naive_projection(conv1d):
    N, T, n_in, n_out, k_i, k_o = 4, 3, 6, 5, 3, 2
    if conv1d:
        transformers = pytest.importorskip("transformers")
        layer = transformers.pytorch_utils.Conv1D(n_out, n_in).double()
        P_i = randn((k_i, n_out), 17).double()   # acts on the output-grad side
        P_o = randn((k_o, n_in), 18).double()
    else:
        layer = nn.Linear(n_in, n_out).double()
        P_i = randn((k_i, n_in), 17).double()
        P_o = randn((k_o, n_out), 18).double()
    X = randn((N, T, n_in), 19).double()
    head = _head(20, n_out).double()
    A, B = _run_layer(layer, X, head, N)
    # per-sample gradients of the summed per-sample loss (the reference multiplies by B)
    g = brute.per_sample_grads(layer, X, X, _sample_loss(head), 1.0)["weight"]
    if conv1d:   # Conv1D weight [n_in, n_out]; block stored [k_i, k_o] = P_i W^T P_o^T
        naive = torch.einsum('ip,bdp,od->bio', P_i, g, P_o)
    else:        # naive check of Examples/ghost_gradproj_mlp.py:37-90: P_o W P_i^T
        naive = torch.einsum('op,bpd,id->boi', P_o, g, P_i)
    assert_close(R.kron_proj_exact(A, B, P_i, P_o, float(N), conv1d=conv1d), naive, 1e-10,
                 "exact")
    assert_close(R.kron_proj_ref(A, B, P_i, P_o, conv1d=conv1d).double(), naive, 1e-6, "ref")
    assert_close(R.kron_proj_projfirst_exact(A, B, P_i, P_o, float(N), conv1d=conv1d), naive,
                 1e-10, "projection first")


def test_embedding_projection_forms_match_per_sample_gradients():
    N, T, V, d, k_i, k_o = 3, 7, 11, 5, 4, 3
    emb = nn.Embedding(V, d).double()
    ids = torch.randint(0, V, (N, T), generator=gen(23))
    ids[0, :4] = 2                         # repeated ids within a sample
    head = _head(24, d).double()
    P_i = randn((k_i, V), 25).double()
    P_o = randn((k_o, d), 26).double()
    out = emb(ids)
    out.retain_grad()
    (out * head).sum().backward()
    g = out.grad                           # [N, T, d]
    W = brute.per_sample_grads(emb, ids, ids, lambda m, x, y: (m(x) * head).sum(), 1.0)["weight"]
    naive = torch.einsum('od,bvd,iv->boi', P_o, W, P_i)     # P_o W_b^T P_i^T
    assert_close(R.kron_embed_proj_exact(ids, g, P_i, P_o), naive, 1e-10, "exact")
    assert_close(R.kron_embed_proj_ref(ids, g.float(), P_i.float(), P_o.float()).double(),
                 naive, 1e-6, "reference loop")
    # an embedding is a Linear layer on one-hot inputs: the dense identity gives the same
    onehot = torch.nn.functional.one_hot(ids, V).double()
    assert_close(R.kron_proj_exact(onehot, g, P_i, P_o, 1.0), naive, 1e-10, "one-hot dense")
    assert_close(R.kron_embed_proj_projfirst_exact(ids, g, P_i, P_o), naive, 1e-10,
                 "projection first")


# ------------------------------------------------------------------ Conv2d
CONV = dict(kernel_size=(3, 2), dilation=(1, 2), padding=(1, 0), stride=(2, 1))


def test_conv2d_forms_match_per_sample_gradients():
    N, n_val, C, H, W, P = 5, 1, 3, 7, 6, 4
    layer = nn.Conv2d(C, P, **CONV).double()
    X = randn((N, C, H, W), 51).double()
    head = randn((P,), 52).double().view(1, P, 1, 1)

    def loss(m, x, y):
        return (torch.tanh(m(x)) * head).sum()

    cap = Capture(layer)
    layer.zero_grad()
    (torch.tanh(layer(X)) * head).reshape(N, -1).sum(1).sum().backward()
    A, B = cap.A, cap.B
    g = brute.per_sample_grads(layer, X, X, loss, 1.0)
    # n_val = 1: the presum dot is <g_i, g_val>
    assert_close(R.conv2d_dot_exact(A, B, n_val, CONV), brute.pairwise_dots(g["weight"], n_val),
                 1e-10, "conv2d weight")
    w_ref, b_ref = R.conv2d_dot_ref(A.float(), B.float(), n_val, CONV)
    assert_close(w_ref.double(), brute.pairwise_dots(g["weight"], n_val), BF16_TOL, "conv2d ref")
    assert_close(b_ref.double(), brute.pairwise_dots(g["bias"], n_val), BF16_TOL, "conv2d bias")
    assert_close(R.bias_dot_exact(B.double().flatten(2).transpose(1, 2), n_val),
                 brute.pairwise_dots(g["bias"], n_val), 1e-10, "conv2d bias exact")


@pytest.mark.parametrize("n_val", [1, 2])
def test_conv2d_ghost_branch_forms(n_val):
    """The reference's Conv2d ghost-branch quantity (defined when C_in*kh*kw == C_out):
    conv2d_ghost_exact's [L, L] cross-Gram contraction against the Gram-Hadamard sum written
    as explicit loops, and the bf16 op sequence against both."""
    import torch.nn.functional as F
    N, C, H, W = 4 + n_val, 2, 7, 6
    i = C * 3 * 2
    X = randn((N, C, H, W), 53).double()
    A_u = F.unfold(X, **CONV)                                  # [N, i, L]
    L = A_u.size(2)
    B = randn((N, i, L), 54).double().reshape(N, i, 4, L // 4)  # a C_out = i backprop
    n_t = N - n_val
    Abar, Bbar = A_u[n_t:].sum(0), B.reshape(N, i, L)[n_t:].sum(0)
    want = torch.zeros(n_t, dtype=torch.float64)
    for b in range(n_t):
        Ab, Bb = A_u[b], B[b].reshape(i, L)
        for x in range(i):
            for y in range(i):
                aa = sum(Abar[x, k] * Ab[y, k] for k in range(L))
                bb = sum(Bbar[x, k] * Bb[y, k] for k in range(L))
                want[b] += aa * bb
    assert_close(R.conv2d_ghost_exact(X, B, n_val, CONV), want, 1e-10, "cross-Gram form")
    assert_close(R.conv2d_ghost_ref(X.float(), B.float(), n_val, CONV).double(), want,
                 BF16_TOL, "bf16 op sequence")
    # Not the presum dot of the per-sample gradients (the quantity both branches aim at).
    presum = R.conv2d_dot_exact(X, B, n_val, CONV)
    assert (presum - want).abs().max() > 1e-3 * want.abs().max()


def test_conv2d_presum_by_explicit_position_loops():
    """n_val = 2: dot_i = sum_{l,m} <a_il, abar_m> <b_il, bbar_m> over unfolded positions."""
    N, n_val, C, H, W, P = 4, 2, 2, 5, 4, 3
    A = randn((N, C, H, W), 53).double()
    Hout = (H + 2 * 1 - 1 * (3 - 1) - 1) // 2 + 1
    Wout = (W + 2 * 0 - 2 * (2 - 1) - 1) // 1 + 1
    B = randn((N, P, Hout, Wout), 54).double()
    a = torch.nn.functional.unfold(A, **CONV)       # [N, d, L]
    b = B.reshape(N, P, -1)
    n_t = N - n_val
    abar, bbar = a[n_t:].sum(0), b[n_t:].sum(0)
    want = torch.zeros(n_t, dtype=torch.float64)
    for i in range(n_t):
        for l in range(a.shape[-1]):
            for m in range(a.shape[-1]):
                want[i] += (a[i, :, l] @ abar[:, m]) * (b[i, :, l] @ bbar[:, m])
    assert_close(R.conv2d_dot_exact(A, B, n_val, CONV), want, 1e-10, "conv2d presum loops")


def test_choose_ki_ko_known_answers():
    # GPT-2-medium shapes, k_total=256, k_min=8 (engine_manager defaults): values obtained
    # by hand from projection_utils.py:12-66.
    cases = {(1024, 3072): (28, 9), (3072, 1024): (9, 28), (1024, 4096): (32, 8),
             (4096, 1024): (8, 32), (1024, 1024): (16, 16)}
    for (n_i, n_o), want in cases.items():
        assert R.choose_ki_ko(n_i, n_o, 256, 8) == want
    with pytest.raises(ValueError):
        R.choose_ki_ko(4, 4, 16, 8)
    with pytest.raises(ValueError):
        R.choose_ki_ko(0, 4, 16, 1)


def test_ghost_switch_decisions_at_baseline_shapes():
    # Linear microbench: ghost for T <= 1024, materialised at T = 2048
    for T, want in [(128, True), (512, True), (1024, True), (2048, False)]:
        assert R.should_use_ghost(T, 768 * 3072) is want
    # GPT-2-small at T=1024: qkv, proj materialise; fc, fc_out, lm_head ghost
    for numel, want in [(768 * 2304, False), (768 * 768, False), (768 * 3072, True),
                        (3072 * 768, True), (50257 * 768, True)]:
        assert R.should_use_ghost(1024, numel) is want
    assert R.tokens(torch.zeros(3, 7)) == 1
    assert R.tokens(torch.zeros(3, 2, 5, 7)) == 10


def test_normwise_check_rejects_planted_errors():
    y = randn((64,), 21).double()
    x = y.clone()
    x[5] += 0.03 * y.abs().max()
    ok, _ = R.normwise_close(x, y, 2e-2)
    assert not ok
    ok, _ = R.normwise_close(y * (1 + 1e-3), y, 2e-2)
    assert ok
    # a transposed operand in the closed form is caught by the brute-force comparison
    A = randn((5, 3, 4), 22).double()
    B = randn((5, 3, 4), 23).double()
    ok, _ = R.normwise_close(R.linear_dot_exact(B, A, 2), R.linear_dot_exact(A, B, 2), 1e-6)
    assert ok  # <G, G'> is symmetric in (A, B) swap ... but the pair of roles matters below
    bad = R.linear_dot_exact(A.flip(1), B, 2)
    ok, _ = R.normwise_close(bad, R.linear_dot_exact(A, B, 2), 1e-6)
    assert not ok
