"""GPU parity of the Linear weight/bias dot kernels against the oracle (through the C ABI).

Tolerances: bf16 operands 2e-2 normwise, fp32 operands 1e-4 normwise, both against the
float64 closed forms; the ghost kernel with reference rounding against the reference's
own bf16 op sequence at 2e-3.
"""
import pytest
import torch

from ghostsuite_amd import _native
from oracle import ghost_ref as R
from tests.helpers import BF16_TOL, FP32_TOL, assert_close, randn

pytestmark = pytest.mark.gpu

SHAPES = [
    # N, n_val, T, d_in, d_out
    (6, 2, 5, 24, 40),        # ragged everything, K tails below one tile
    (10, 3, 64, 128, 96),
    (80, 16, 1, 512, 1024),   # the MLP layer shape (T = 1)
    (8, 2, 300, 200, 136),    # T and K not multiples of the tile sizes
    (12, 4, 130, 64, 10),     # d_out = 10: unaligned rows, scalar loads
    (6, 2, 256, 128, 192),    # T a multiple of the tile width: per-tile partial sums
]


def _inputs(N, T, d_in, d_out, seed, dtype):
    A = randn((N, T, d_in), seed, 1.0, dtype)
    G = randn((N, T, d_out), seed + 1, 1e-3, dtype)
    return A, G


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("algo", [_native.ALGO_GHOST, _native.ALGO_VALGRAD])
@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
def test_linear_dot_matches_closed_form(gpu, shape, dtype, algo, semantics):
    N, n_val, T, d_in, d_out = shape
    print(f"linear_dot shape={shape} dtype={dtype} algo={algo} sem={semantics}", flush=True)
    A, G = _inputs(N, T, d_in, d_out, 100 + N + T, dtype)
    sem = _native.SEM_PAIRWISE_SUM if semantics == "pairwise" else _native.SEM_PRESUM
    dot, _ = _native.ops().linear_dot(A.to(gpu), G.to(gpu), n_val, semantics=sem, algo=algo)
    torch.cuda.synchronize()
    want = R.linear_dot_exact(A, G, n_val, semantics)
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert_close(dot.cpu(), want, tol, f"{semantics}/{algo}")


@pytest.mark.parametrize("shape", SHAPES[:4])
@pytest.mark.parametrize("algo", [_native.ALGO_GHOST, _native.ALGO_VALGRAD])
def test_linear_pairs_and_val_first_layout(gpu, shape, algo):
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 7 + T, torch.float32)
    for val_start in (0, N - n_val, 1):
        if val_start + n_val > N:
            continue
        print(f"pairs shape={shape} algo={algo} val_start={val_start}", flush=True)
        dot, pair = _native.ops().linear_dot(A.to(gpu), G.to(gpu), n_val, val_start=val_start,
                                             algo=algo, want_pair=True)
        torch.cuda.synchronize()
        want_pair = R.linear_dot_exact(A, G, n_val, "pairwise", val_start=val_start, pair=True)
        want_dot = R.linear_dot_exact(A, G, n_val, "pairwise", val_start=val_start)
        assert_close(pair.cpu(), want_pair, FP32_TOL, "pair")
        assert_close(dot.cpu(), want_dot, FP32_TOL, "dot")
        # invariant: summing the pair matrix over val rows gives the dot vector
        assert_close(pair.cpu().double().sum(0), dot.cpu().double(), 1e-5, "pair-sum")


@pytest.mark.parametrize("shape", [(10, 3, 64, 128, 96), (6, 2, 40, 64, 72)])
def test_ghost_reference_rounding_matches_reference_sequence(gpu, shape):
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 31, torch.float32)
    dot, _ = _native.ops().linear_dot(A.to(gpu).bfloat16(), G.to(gpu).bfloat16(), n_val,
                                      algo=_native.ALGO_GHOST,
                                      rounding=_native.ROUND_REF_BF16)
    torch.cuda.synchronize()
    want, _ = R.linear_dot_ref(A, G, n_val, use_ghost=True, has_bias=False)
    assert_close(dot.cpu(), want, 2e-3, "ref-rounding")


@pytest.mark.parametrize("shape,pair", [((32, 8, 1024, 64, 96), False),   # per-tile partials
                                        ((20, 5, 600, 40, 72), False),    # per-token, K tails
                                        ((40, 10, 512, 32, 48), True)])   # per val row
def test_ghost_many_tiles(gpu, shape, pair):
    """Grids of 400-3000 tiles (several waves of workgroups per CU, both partial layouts, K
    tails, per-val-row tiles): bf16 dots (and per-pair values) against the float64 closed
    form."""
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 500 + T, torch.bfloat16)
    print(f"ghost many tiles shape={shape} pair={pair}", flush=True)
    dot, prs = _native.ops().linear_dot(A.to(gpu), G.to(gpu), n_val, algo=_native.ALGO_GHOST,
                                        want_pair=pair)
    torch.cuda.synchronize()
    Af, Gf = A.float(), G.float()
    assert_close(dot.cpu(), R.linear_dot_exact(Af, Gf, n_val, "pairwise"), BF16_TOL, "dot")
    if pair:
        assert_close(prs.cpu(), R.linear_dot_exact(Af, Gf, n_val, "pairwise", pair=True),
                     BF16_TOL, "pair")


def test_ghost_many_tiles_reference_rounding(gpu):
    N, n_val, T, d_in, d_out = 20, 5, 600, 40, 72
    A, G = _inputs(N, T, d_in, d_out, 77, torch.float32)
    dot, _ = _native.ops().linear_dot(A.to(gpu).bfloat16(), G.to(gpu).bfloat16(), n_val,
                                      algo=_native.ALGO_GHOST,
                                      rounding=_native.ROUND_REF_BF16)
    torch.cuda.synchronize()
    want, _ = R.linear_dot_ref(A, G, n_val, use_ghost=True, has_bias=False)
    assert_close(dot.cpu(), want, 2e-3, "ref-rounding")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_linear_rowdot_with_given_v(gpu, shape, dtype):
    """gs_linear_rowdot: sum_t g_it^T V a_it for a caller-formed V, at a val block in the
    middle of the batch."""
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 300 + T, dtype)
    V = randn((d_out, d_in), 301 + T, 1.0, dtype)
    vs = 1 if N - n_val >= 1 else 0
    print(f"rowdot shape={shape} dtype={dtype}", flush=True)
    out = _native.ops().linear_rowdot(A.to(gpu), G.to(gpu), V.to(gpu), n_val, val_start=vs)
    torch.cuda.synchronize()
    tr = torch.cat([A[:vs], A[vs + n_val:]]).double().reshape(N - n_val, -1, d_in)
    gt = torch.cat([G[:vs], G[vs + n_val:]]).double().reshape(N - n_val, -1, d_out)
    want = torch.einsum('ntp,pd,ntd->n', gt, V.double(), tr)
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert_close(out.cpu(), want, tol, "rowdot")


def test_linear_auto_picks_cheaper_algorithm(gpu):
    ops = _native.ops()
    # microbench T=1024: ghost 1.5 TF vs val-gradient 0.15 TF
    assert ops.linear_algo(torch.bfloat16, 32, 8, 1024, 768, 3072, 0, 0,
                           False) == _native.ALGO_VALGRAD
    # tiny T with big layers: ghost
    assert ops.linear_algo(torch.bfloat16, 20, 4, 4, 1024, 4096, 0, 0, False) == _native.ALGO_GHOST


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(6, 2, 5, 40), (10, 3, 130, 96), (80, 16, 1, 10),
                                   (6, 2, 40, 3072), (4, 1, 33, 1030), (20, 4, 1024, 768),
                                   (10, 2, 2048, 8192)])
@pytest.mark.parametrize("mid", [False, True])
def test_bias_dot_and_grad(gpu, dtype, shape, mid):
    """Bias dots and train grad against float64; `mid`: the val block between train rows
    (the oracle sees the same samples with the val block moved to the end)."""
    N, n_val, T, d = shape
    G = randn((N, T, d), 5 + T, 1e-3, dtype)
    scale = N / (N - n_val)
    vs = 1 if mid else N - n_val
    print(f"bias shape={shape} dtype={dtype} val_start={vs}", flush=True)
    dot, grad = _native.ops().bias_dot(G.to(gpu), n_val, val_start=vs, grad_scale=scale,
                                       grad_dtype=torch.float32)
    torch.cuda.synchronize()
    Go = torch.cat([G[:vs], G[vs + n_val:], G[vs:vs + n_val]])  # val rows last
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert_close(dot.cpu(), R.bias_dot_exact(Go, n_val), tol, "bias dot")
    want_grad = R.bias_train_grad(Go.double() * N, n_val)
    assert_close(grad.cpu(), want_grad, tol, "bias grad")


def test_linear_rejects_bad_arguments(gpu):
    A = torch.zeros(4, 3, 8, device=gpu)
    G = torch.zeros(4, 3, 8, device=gpu)
    with pytest.raises(_native.GhostHipError):
        _native.ops().linear_dot(A, G, 4)            # no train rows
    with pytest.raises(_native.GhostHipError):
        _native.ops().linear_dot(A, G.bfloat16(), 1)  # dtype mismatch
    with pytest.raises(_native.GhostHipError):
        _native.ops().linear_dot(A, G, 1, semantics=_native.SEM_PRESUM, want_pair=True)


@pytest.mark.parametrize("shape", SHAPES + [(8, 4, 512, 256, 512), (5, 2, 1024, 768, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
def test_linear_val_gradient_matches_closed_form(gpu, shape, dtype, semantics):
    N, n_val, T, d_in, d_out = shape
    print(f"linear_val_gradient shape={shape} dtype={dtype} sem={semantics}", flush=True)
    A, G = _inputs(N, T, d_in, d_out, 300 + N + T, dtype)
    sem = _native.SEM_PAIRWISE_SUM if semantics == "pairwise" else _native.SEM_PRESUM
    V = _native.ops().linear_val_gradient(A.to(gpu), G.to(gpu), n_val, val_start=1,
                                          semantics=sem)
    torch.cuda.synchronize()
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert V.shape == (d_out, d_in) and V.dtype == dtype
    assert_close(V.cpu().double(), R.val_term_exact(A, G, n_val, semantics, val_start=1), tol,
                 f"val term {semantics}")


@pytest.mark.parametrize("shape", [(6, 2, 256, 128, 256), (5, 1, 512, 64, 512),
                                   (4, 1, 256, 768, 768)])
@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
@pytest.mark.parametrize("caller_v", [False, True])
def test_linear_bias_fused_matches_closed_forms(gpu, caller_v, shape, semantics):
    """Weight dot, bias dot and bias train gradient in one pass: gs_linear_bias_dot, and
    gs_linear_rowdot_bias with a V the caller formed (here a float64 val term rounded to
    bf16)."""
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 400 + T, torch.bfloat16)
    scale = N / (N - n_val) / 7.0
    print(f"linear_bias_dot shape={shape} sem={semantics} caller_v={caller_v}", flush=True)
    sem = _native.SEM_PAIRWISE_SUM if semantics == "pairwise" else _native.SEM_PRESUM
    if caller_v:
        V = R.val_term_exact(A, G, n_val, semantics).to(torch.bfloat16)
        res = _native.ops().linear_rowdot_bias(A.to(gpu), G.to(gpu), V.to(gpu), n_val,
                                               grad_scale=scale, grad_dtype=torch.float32)
    else:
        res = _native.ops().linear_bias_dot(A.to(gpu), G.to(gpu), n_val, semantics=sem,
                                            algo=_native.ALGO_VALGRAD, grad_scale=scale,
                                            grad_dtype=torch.float32)
    assert res is not None
    dot, bdot, bgrad = res
    torch.cuda.synchronize()
    assert_close(dot.cpu(), R.linear_dot_exact(A, G, n_val, semantics), BF16_TOL, "weight dot")
    assert_close(bdot.cpu(), R.bias_dot_exact(G, n_val), BF16_TOL, "bias dot")
    assert_close(bgrad.cpu(), R.bias_train_grad(G.double() * N, n_val) * (1 / 7.0), BF16_TOL,
                 "bias grad")


@pytest.mark.parametrize("shape", [(20, 4, 1024, 64, 768), (20, 4, 1024, 32, 2304)])
@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
def test_rowdot_192_row_tiles(gpu, shape, semantics):
    """d_out 768 and 2304 over 64 train-token tiles: the row-dot takes 192-row tiles (256 and
    768 workgroups instead of 192 and 576), for the plain dot and the fused bias pass."""
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 600 + d_out, torch.bfloat16)
    sem = _native.SEM_PAIRWISE_SUM if semantics == "pairwise" else _native.SEM_PRESUM
    print(f"rowdot 192 shape={shape} sem={semantics}", flush=True)
    ops = _native.ops()
    dot, _ = ops.linear_dot(A.to(gpu), G.to(gpu), n_val, semantics=sem, algo=_native.ALGO_VALGRAD)
    dot2, bdot, bgrad = ops.linear_bias_dot(A.to(gpu), G.to(gpu), n_val, semantics=sem,
                                            algo=_native.ALGO_VALGRAD,
                                            grad_scale=N / (N - n_val), grad_dtype=torch.float32)
    torch.cuda.synchronize()
    want = R.linear_dot_exact(A, G, n_val, semantics)
    assert_close(dot.cpu(), want, BF16_TOL, "weight dot")
    assert_close(dot2.cpu(), want, BF16_TOL, "weight dot (fused)")
    assert_close(bdot.cpu(), R.bias_dot_exact(G, n_val), BF16_TOL, "bias dot")
    assert_close(bgrad.cpu(), R.bias_train_grad(G.double() * N, n_val), BF16_TOL, "bias grad")


@pytest.mark.parametrize("shape", [(12, 4, 256, 768, 3072), (6, 2, 256, 256, 1000),
                                   (6, 2, 512, 1280, 1536), (82, 2, 256, 768, 1024)])
@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
def test_valgrad_over_d_out(gpu, shape, semantics):
    """d_out > d_in: the val-gradient row-dot runs over K = d_out (V^T, Z = the train rows of
    A) and the fused bias pass sums the train rows of G inside its mainloop.  192-row tiles
    over d_in 768 (each token tile's rows split 64/64/64/64 over 4 workgroups); one 256-row
    tile (all 256 rows in one workgroup, four passes of 64) with a K tail of 40; five 256-row
    tiles (rows split 52/52/52/52/48); three 256-row tiles over 80 token tiles (rows split
    86/86/84: a whole first pass and a partial second one).  Val rows first and last; per-pair
    values for the pairwise sum."""
    N, n_val, T, d_in, d_out = shape
    A, G = _inputs(N, T, d_in, d_out, 700 + d_in, torch.bfloat16)
    sem = _native.SEM_PAIRWISE_SUM if semantics == "pairwise" else _native.SEM_PRESUM
    ops = _native.ops()
    for val_start in (N - n_val, 0):
        print(f"valgrad over d_out shape={shape} sem={semantics} val_start={val_start}",
              flush=True)
        pair = semantics == "pairwise"
        dot, prs = ops.linear_dot(A.to(gpu), G.to(gpu), n_val, val_start=val_start,
                                  semantics=sem, algo=_native.ALGO_VALGRAD, want_pair=pair)
        torch.cuda.synchronize()
        want = R.linear_dot_exact(A, G, n_val, semantics, val_start=val_start)
        assert_close(dot.cpu(), want, BF16_TOL, "weight dot")
        if pair:
            assert_close(prs.cpu(), R.linear_dot_exact(A, G, n_val, "pairwise",
                                                       val_start=val_start, pair=True),
                         BF16_TOL, "pair")
    # The fused weight + bias pass (gs_linear_bias_dot), val rows last and in the middle.
    for val_start in (N - n_val, 1):
        dot2, bdot, bgrad = ops.linear_bias_dot(A.to(gpu), G.to(gpu), n_val, val_start=val_start,
                                                semantics=sem, algo=_native.ALGO_VALGRAD,
                                                grad_scale=N / (N - n_val),
                                                grad_dtype=torch.float32)
        torch.cuda.synchronize()
        assert_close(dot2.cpu(), R.linear_dot_exact(A, G, n_val, semantics, val_start=val_start),
                     BF16_TOL, "weight dot (fused)")
        assert_close(bdot.cpu(), R.bias_dot_exact(G, n_val, val_start=val_start), BF16_TOL,
                     "bias dot")
        tr = torch.cat([G[:val_start], G[val_start + n_val:]]).double()
        assert_close(bgrad.cpu(), tr.sum((0, 1)) * N / (N - n_val), BF16_TOL, "bias grad")


@pytest.mark.parametrize("semantics", ["pairwise", "presum"])
def test_valgrad_over_d_out_unaligned_operands(gpu, semantics):
    """bf16 operands 2 bytes past a 16-byte boundary (through the C ABI; the wrapper would copy
    them): the val-gradient pass takes the transposed-operand path (STORE GEMM for V^T,
    element loads in the row-dot and its epilogue), still over K = d_out."""
    N, n_val, T, d_in, d_out = 6, 2, 64, 64, 160
    A, G = _inputs(N, T, d_in, d_out, 900, torch.bfloat16)
    sem = _native.SEM_PAIRWISE_SUM if semantics == "pairwise" else _native.SEM_PRESUM
    lib = _native.load_library()
    bufs = []
    for t in (A, G):
        b = torch.zeros(t.numel() + 8, dtype=torch.bfloat16, device=gpu)
        b[1:1 + t.numel()] = t.reshape(-1).to(gpu)
        bufs.append(b)
    dev = torch.device(gpu)
    ws_bytes = lib.gs_linear_dot_workspace(_native.DTYPE_BF16, N, n_val, T, d_in, d_out, sem,
                                           _native.ALGO_VALGRAD, 0)
    assert ws_bytes > 0
    ws = _native._workspace(ws_bytes, dev)
    out = torch.empty(N - n_val, dtype=torch.float32, device=gpu)
    print(f"valgrad unaligned sem={semantics}", flush=True)
    rc = lib.gs_linear_dot(bufs[0].data_ptr() + 2, bufs[1].data_ptr() + 2, _native.DTYPE_BF16,
                           N, n_val, N - n_val, T, d_in, d_out, sem, _native.ALGO_VALGRAD,
                           _native.ROUND_FP32, out.data_ptr(), None, ws.data_ptr(), ws_bytes,
                           _native._stream(dev))
    assert rc == 0, lib.gs_last_error()
    torch.cuda.synchronize()
    assert_close(out.cpu(), R.linear_dot_exact(A, G, n_val, semantics), BF16_TOL, "dot")


def test_linear_bias_fused_declines_unsupported_shapes(gpu):
    ops = _native.ops()
    A, G = _inputs(6, 100, 64, 256, 5, torch.bfloat16)        # T not a multiple of 256
    assert ops.linear_bias_dot(A.to(gpu), G.to(gpu), 2, algo=_native.ALGO_VALGRAD) is None
    A, G = _inputs(6, 256, 64, 200, 6, torch.bfloat16)        # d_out not a multiple of 192/256
    assert ops.linear_bias_dot(A.to(gpu), G.to(gpu), 2, algo=_native.ALGO_VALGRAD) is None
    A, G = _inputs(6, 256, 64, 256, 7, torch.float32)         # fp32 operands
    assert ops.linear_bias_dot(A.to(gpu), G.to(gpu), 2, algo=_native.ALGO_VALGRAD) is None


def _train_grad_want(A, G, n_val, vs, scale, conv1d, dev):
    """float64 reference on the device: scale * sum over the train rows of g a^T (or a g^T)."""
    N = A.shape[0]
    keep = [i for i in range(N) if not vs <= i < vs + n_val]
    a = A[keep].to(dev, torch.float64).reshape(-1, A.shape[-1])
    g = G[keep].to(dev, torch.float64).reshape(-1, G.shape[-1])
    w = (a.t() @ g) if conv1d else (g.t() @ a)
    return (w * scale).cpu()


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", [
    # N, n_val, T, d_in, d_out, val position
    (6, 2, 33, 40, 24, "last"), (6, 2, 33, 40, 24, "first"), (6, 2, 33, 40, 24, "mid"),
    (3, 1, 1, 8, 16, "mid"), (5, 1, 300, 136, 264, "mid"),
    (20, 4, 1024, 768, 3072, "last"), (20, 4, 1024, 3072, 768, "last"),
    (20, 4, 1024, 768, 2304, "mid"), (20, 4, 1024, 768, 768, "first"),
    (10, 2, 2048, 2048, 8192, "last"),
    # 256 or more 256 x 256 output tiles: the wide-tile kernel (edge tiles, val block inside)
    (3, 1, 256, 4104, 4096, "mid"), (4, 2, 192, 8192, 2056, "first"),
])
@pytest.mark.parametrize("conv1d", [False, True])
def test_linear_train_grad(gpu, out_dtype, case, conv1d):
    """gs_linear_train_grad (K-major GEMM over the train rows, val block skipped) against a
    float64 product; at bf16 output the one rounding is the only error."""
    N, n_val, T, d_in, d_out, pos = case
    vs = {"last": N - n_val, "first": 0, "mid": 1}[pos]
    A = randn((N, T, d_in), 90 + T, 1.0, torch.bfloat16)
    G = randn((N, T, d_out), 91 + T, 1e-3, torch.bfloat16)
    scale = 1.25 / (N - n_val)
    print(f"train grad case={case} out={out_dtype} conv1d={conv1d}", flush=True)
    out = _native.ops().linear_train_grad(A.to(gpu), G.to(gpu), n_val, scale, val_start=vs,
                                          out_dtype=out_dtype, conv1d=conv1d)
    assert out is not None and out.dtype == out_dtype
    assert tuple(out.shape) == ((d_in, d_out) if conv1d else (d_out, d_in))
    want = _train_grad_want(A, G, n_val, vs, scale, conv1d, gpu)
    tol = 1e-2 if out_dtype == torch.bfloat16 else FP32_TOL
    assert_close(out.cpu(), want, tol, "train grad")


def test_linear_train_grad_declines_and_sampler_falls_back(gpu):
    """Cases outside the kernel return None (fp32 operands, feature counts not multiples of 8);
    the Linear sampler then takes the addmm path, and at a supported shape its result is the
    kernel's."""
    from ghostsuite_amd.supported_layers_grad_samplers_dotprod import _compute_linear_train_grad
    ops = _native.ops()
    A = randn((4, 16, 40), 95, 1.0, torch.float32).to(gpu)
    G = randn((4, 16, 24), 96, 1e-3, torch.float32).to(gpu)
    assert ops.linear_train_grad(A, G, 1, 0.5) is None
    A2 = randn((4, 16, 12), 97, 1.0, torch.bfloat16).to(gpu)
    G2 = randn((4, 16, 24), 98, 1e-3, torch.bfloat16).to(gpu)
    assert ops.linear_train_grad(A2, G2, 1, 0.5) is None
    layer = torch.nn.Linear(12, 24)
    for a, g in ((A, G), (A2, G2)):
        got = _compute_linear_train_grad(layer, a, g, 1, scale=2.0)
        want = _train_grad_want(a.cpu(), g.cpu(), 1, 3, 2.0 / 3, False, gpu)
        assert_close(got.float().cpu(), want, 1e-2, "sampler fallback")
    A3 = randn((4, 32, 40), 99, 1.0, torch.bfloat16).to(gpu)
    G3 = randn((4, 32, 24), 100, 1e-3, torch.bfloat16).to(gpu)
    bf16 = dict(dtype=torch.bfloat16)
    got = _compute_linear_train_grad(torch.nn.Linear(40, 24, **bf16), A3, G3, 1, scale=2.0)
    assert torch.equal(got, ops.linear_train_grad(A3, G3, 1, 2.0 / 3))
    # An fp32 parameter with bf16 operands (autocast): the gradient in the parameter's dtype.
    got = _compute_linear_train_grad(torch.nn.Linear(40, 24), A3, G3, 1, scale=2.0)
    assert got.dtype == torch.float32
    assert torch.equal(got, ops.linear_train_grad(A3, G3, 1, 2.0 / 3, out_dtype=torch.float32))
    # 256 to 1023 output tiles of 128 x 128: hipBLASLt through addmm (faster there).
    from ghostsuite_amd.supported_layers_grad_samplers_dotprod import _scaled_mm
    A4 = randn((3, 8, 2048), 101, 1.0, torch.bfloat16).to(gpu)
    G4 = randn((3, 8, 2048), 102, 1e-3, torch.bfloat16).to(gpu)
    got = _compute_linear_train_grad(torch.nn.Linear(2048, 2048, **bf16), A4, G4, 1, scale=2.0)
    want = _scaled_mm(G4[:2].reshape(-1, 2048).t(), A4[:2].reshape(-1, 2048), 1.0)
    assert torch.equal(got, want)
    # 256 tiles of 256 x 256 and more: the wide-tile kernel again.
    A5 = randn((3, 16, 2048), 103, 1.0, torch.bfloat16).to(gpu)
    G5 = randn((3, 16, 8192), 104, 1e-3, torch.bfloat16).to(gpu)
    got = _compute_linear_train_grad(torch.nn.Linear(2048, 8192, **bf16), A5, G5, 1, scale=2.0)
    assert torch.equal(got, ops.linear_train_grad(A5, G5, 1, 2.0 / 2))


@pytest.mark.parametrize("case", [
    # N, n_val, T, d_in, d_out, semantics, val position, bias
    (6, 2, 64, 40, 24, "pairwise", "last", True),
    (6, 2, 64, 40, 24, "presum", "mid", True),
    (6, 2, 128, 136, 264, "pairwise", "first", False),
    (3, 2, 64, 16, 8, "presum", "last", True),           # one train row
    (7, 1, 192, 264, 136, "pairwise", "mid", True),
    (20, 4, 1024, 768, 3072, "pairwise", "last", True),  # GPT-2-small fc
    (20, 4, 1024, 3072, 768, "pairwise", "last", True),  # fc_out
    (20, 4, 1024, 768, 2304, "presum", "last", True),    # qkv
    (20, 4, 1024, 768, 768, "presum", "mid", True),      # proj
    (10, 2, 2048, 2048, 8192, "pairwise", "last", True),  # Pythia-1B fc
    # splits that start and end inside samples (k-rows per split 1.33 and 2.6 samples), and
    # a split estimate below one sample (raised to one sample per split)
    (9, 1, 192, 512, 512, "presum", "last", True),
    (12, 2, 320, 1024, 1024, "pairwise", "first", True),
    (5, 1, 1024, 136, 264, "pairwise", "mid", True),
    # 256 x 256 train-row tiles (224 tiles and more): whole, and cut by the matrix edges on
    # both sides, with and without the bias terms
    (4, 1, 64, 2048, 7168, "pairwise", "mid", True),
    (4, 1, 64, 2000, 7176, "presum", "first", True),
    (4, 2, 64, 7176, 2000, "pairwise", "last", False),
])
@pytest.mark.parametrize("grad_dtype", [torch.bfloat16, torch.float32])
def test_linear_dot_train_grad(gpu, case, grad_dtype):
    """gs_linear_dot_train_grad (one K-major pass over the train rows: dots at the sample
    boundaries, the train gradient from the same accumulators, per-sample column sums of G
    for the bias) against float64: dots through the val-term form, the weight and bias
    train gradients as closed forms."""
    N, n_val, T, d_in, d_out, sem, pos, bias = case
    vs = {"last": N - n_val, "first": 0, "mid": 1}[pos]
    A = randn((N, T, d_in), 110 + T, 1.0, torch.bfloat16)
    G = randn((N, T, d_out), 111 + T, 1e-3, torch.bfloat16)
    n_t = N - n_val
    semantics = _native.SEM_PAIRWISE_SUM if sem == "pairwise" else _native.SEM_PRESUM
    print(f"dot+train grad case={case} grad={grad_dtype}", flush=True)
    Ad, Gd = A.to(gpu), G.to(gpu)
    res = _native.ops().linear_dot_train_grad(
        Ad, Gd, n_val, val_start=vs, semantics=semantics, grad_scale=1.5 / n_t,
        grad_dtype=grad_dtype, bias=bias, bias_grad_scale=0.75 / n_t, bias_grad_dtype=grad_dtype)
    assert res is not None
    dot, grad, bdot, bgrad = res
    want_dot = R.linear_dot_valterm_exact(Ad, Gd, n_val, sem, val_start=vs).cpu()
    assert_close(dot.cpu(), want_dot, BF16_TOL, "weight dot")
    tol = 1e-2 if grad_dtype == torch.bfloat16 else FP32_TOL
    assert_close(grad.float().cpu(), _train_grad_want(A, G, n_val, vs, 1.5 / n_t, False, gpu),
                 tol, "weight train grad")
    if bias:
        assert_close(bdot.cpu(), R.bias_dot_exact(G, n_val, vs), BF16_TOL, "bias dot")
        tr, _ = R.split_rows(G.double().reshape(N, T, d_out), n_val, vs)
        assert_close(bgrad.float().cpu(), tr.sum((0, 1)) * (0.75 / n_t), tol, "bias train grad")
    else:
        assert bdot is None and bgrad is None


def test_linear_dot_train_grad_declines(gpu):
    ops = _native.ops()
    A, G = _inputs(6, 100, 64, 256, 5, torch.bfloat16)        # T not a multiple of 64
    assert ops.linear_dot_train_grad(A.to(gpu), G.to(gpu), 2, grad_scale=1.0) is None
    A, G = _inputs(6, 64, 12, 256, 6, torch.bfloat16)         # d_in not a multiple of 8
    assert ops.linear_dot_train_grad(A.to(gpu), G.to(gpu), 2, grad_scale=1.0) is None
    A, G = _inputs(6, 64, 64, 256, 7, torch.float32)          # fp32 operands
    assert ops.linear_dot_train_grad(A.to(gpu), G.to(gpu), 2, grad_scale=1.0) is None


@pytest.mark.parametrize("case", [
    # N, n_val, T, d_in, d_out
    (6, 2, 128, 136, 264),
    (20, 4, 1024, 768, 3072),    # GPT-2-small mlp.c_fc
])
def test_conv1d_sampler_fused_dot_and_train_grad(gpu, case):
    """HF Conv1D (weight [d_in, d_out]) takes the fused pass through its own entry point (the
    operands swapped inside): the presum dots, the [d_in, d_out] train gradient and the bias
    dot and train gradient against float64 closed forms, and the same dots as the unfused
    path."""
    transformers = pytest.importorskip("transformers")
    from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
    N, n_val, T, d_in, d_out = case
    n_t = N - n_val
    print(f"conv1d fused case={case}", flush=True)
    layer = transformers.pytorch_utils.Conv1D(d_out, d_in).to(gpu, torch.bfloat16)
    for p in layer.parameters():
        p.initially_requires_grad = True
    A = randn((N, T, d_in), 120, 1.0, torch.bfloat16)
    G = randn((N, T, d_out), 121, 1e-3, torch.bfloat16)
    Ad, Gd = A.to(gpu), G.to(gpu)
    layer._gs_bias_grad_scale = 1.5 / n_t
    S._compute_Conv1D_dot_product(layer, Ad, Gd, n_val)
    assert "_gs_weight_train_grad" in layer.__dict__          # the fused pass ran
    dot = layer.weight.grad_dot_prod.cpu()
    want_dot = R.linear_dot_valterm_exact(Ad, Gd, n_val, "presum").cpu()
    assert_close(dot, want_dot, BF16_TOL, "weight dot")
    grad = S._compute_Conv1D_train_grad(layer, Ad, Gd, n_val, scale=1.5)
    assert grad.shape == (d_in, d_out)
    assert_close(grad.float().cpu(), _train_grad_want(A, G, n_val, N - n_val, 1.5 / n_t, True, gpu),
                 1e-2, "weight train grad")
    assert_close(layer.bias.grad_dot_prod.cpu(), R.bias_dot_exact(G, n_val), BF16_TOL, "bias dot")
    tr, _ = R.split_rows(G.double(), n_val, N - n_val)
    assert_close(layer._gs_bias_train_grad.float().cpu(), tr.sum((0, 1)) * (1.5 / n_t), 1e-2,
                 "bias train grad")
    # without the announced scale the dots come from the unfused path
    del layer._gs_bias_grad_scale
    S._compute_Conv1D_dot_product(layer, Ad, Gd, n_val)
    assert "_gs_weight_train_grad" not in layer.__dict__
    assert_close(layer.weight.grad_dot_prod.cpu(), dot, BF16_TOL, "unfused weight dot")


def _random_fused_cases(n, seed):
    """Seeded shapes inside the fused op's domain: T a multiple of 64, feature counts
    multiples of 8, 1-4 val rows anywhere in the batch, both semantics, with and without a
    bias; sizes kept small enough for float64 checks in seconds."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    cases = []
    for _ in range(n):
        n_val = pick(1, 4)
        N = n_val + pick(1, 6)
        T = 64 * pick(1, 6)
        d_in, d_out = 8 * pick(1, 64), 8 * pick(1, 64)
        vs = pick(0, N - n_val)
        sem = "presum" if pick(0, 1) else "pairwise"
        cases.append((N, n_val, vs, T, d_in, d_out, sem, bool(pick(0, 1))))
    return cases


def _wide_tiles(d_in, d_out):
    """Whether the fused pass takes the train rows in 256 x 256 tiles: 224 of them or more."""
    return -(-d_out // 256) * -(-d_in // 256) >= 224


def _random_wide_cases(n, seed):
    """Seeded shapes of the 256 x 256 train-row tiles: wide feature counts, ragged at both
    edges, and few rows, so the float64 checks stay within seconds."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    cases = []
    while len(cases) < n:
        n_val = pick(1, 2)
        N = n_val + pick(1, 3)
        T = 64
        d_in, d_out = 8 * pick(200, 1000), 8 * pick(200, 1000)
        if not _wide_tiles(d_in, d_out):
            continue
        vs = pick(0, N - n_val)
        sem = "presum" if pick(0, 1) else "pairwise"
        cases.append((N, n_val, vs, T, d_in, d_out, sem, bool(pick(0, 1))))
    return cases


@pytest.mark.parametrize("case", _random_fused_cases(24, 2026) + _random_wide_cases(3, 2027))
def test_linear_dot_train_grad_random_shapes(gpu, case):
    """gs_linear_dot_train_grad over seeded random shapes (split counts, tile edges, cut
    samples and val positions vary together) against the float64 closed forms; the same call
    with the operands swapped (the HF Conv1D path) gives the same dots and the transposed
    train gradient.  The dots are checked against the val-term form with the kernels' bf16
    rounding points (presummed val rows, V): with one or two train rows a dot can be nearly
    orthogonal to V (cos ~ 1e-3 at these sizes), which turns their 0.2% rounding into
    several percent of the dot."""
    N, n_val, vs, T, d_in, d_out, sem, bias = case
    print(f"random fused case={case}", flush=True)
    A = randn((N, T, d_in), 130 + N + T, 1.0, torch.bfloat16)
    G = randn((N, T, d_out), 131 + d_in, 1e-3, torch.bfloat16)
    n_t = N - n_val
    semantics = _native.SEM_PAIRWISE_SUM if sem == "pairwise" else _native.SEM_PRESUM
    Ad, Gd = A.to(gpu), G.to(gpu)
    ops = _native.ops()
    res = ops.linear_dot_train_grad(Ad, Gd, n_val, val_start=vs, semantics=semantics,
                                    grad_scale=1.0 / n_t, grad_dtype=torch.float32, bias=bias,
                                    bias_grad_scale=1.0 / n_t, bias_grad_dtype=torch.float32)
    assert res is not None
    dot, grad, bdot, bgrad = res
    want_dot = R.linear_dot_valterm_exact(Ad, Gd, n_val, sem, val_start=vs,
                                          round_dtype=torch.bfloat16).cpu()
    assert_close(dot.cpu(), want_dot, BF16_TOL, "weight dot")
    want_grad = _train_grad_want(A, G, n_val, vs, 1.0 / n_t, False, gpu)
    assert_close(grad.cpu(), want_grad, FP32_TOL, "weight train grad")
    if bias:
        assert_close(bdot.cpu(), R.bias_dot_exact(G, n_val, vs), BF16_TOL, "bias dot")
        tr, _ = R.split_rows(G.double(), n_val, vs)
        assert_close(bgrad.cpu(), tr.sum((0, 1)) / n_t, FP32_TOL, "bias train grad")
    sw = ops.linear_dot_train_grad(Gd, Ad, n_val, val_start=vs, semantics=semantics,
                                   grad_scale=1.0 / n_t, grad_dtype=torch.float32)
    assert sw is not None
    assert_close(sw[0].cpu(), want_dot, BF16_TOL, "swapped dot")
    assert_close(sw[1].cpu(), want_grad.t(), FP32_TOL, "swapped train grad")
    # the Conv1D entry point: same dots, [d_in, d_out] train gradient, G's bias terms
    cv = ops.linear_dot_train_grad(Ad, Gd, n_val, val_start=vs, semantics=semantics,
                                   grad_scale=1.0 / n_t, grad_dtype=torch.float32, bias=bias,
                                   bias_grad_scale=1.0 / n_t, bias_grad_dtype=torch.float32,
                                   conv1d=True)
    assert cv is not None
    assert_close(cv[0].cpu(), want_dot, BF16_TOL, "conv1d dot")
    assert_close(cv[1].cpu(), want_grad.t(), FP32_TOL, "conv1d train grad")
    if bias:
        assert_close(cv[2].cpu(), R.bias_dot_exact(G, n_val, vs), BF16_TOL, "conv1d bias dot")
        assert_close(cv[3].cpu(), tr.sum((0, 1)) / n_t, FP32_TOL, "conv1d bias train grad")


def _random_dot_cases(n, seed):
    """Seeded shapes for the separate dot and train-gradient entry points: any T, feature
    counts aligned or not (aligned ones take the DMA / K-major kernels, the others the
    transposing path), 1-4 val rows anywhere, at least four train rows (a single near-zero
    dot is then judged against the vector's scale)."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    cases = []
    for _ in range(n):
        n_val = pick(1, 4)
        N = n_val + pick(4, 8)
        T = pick(1, 160)
        d_in = 8 * pick(1, 40) if pick(0, 1) else pick(1, 300)
        d_out = 8 * pick(1, 40) if pick(0, 1) else pick(1, 300)
        cases.append((N, n_val, pick(0, N - n_val), T, d_in, d_out,
                      "presum" if pick(0, 1) else "pairwise",
                      _native.ALGO_GHOST if pick(0, 1) else _native.ALGO_VALGRAD))
    return cases


@pytest.mark.parametrize("case", _random_dot_cases(24, 2027))
def test_linear_dot_random_shapes(gpu, case):
    """gs_linear_dot (ghost and val-gradient algorithms, both semantics) over seeded random
    shapes against the float64 closed form, bf16 operands."""
    N, n_val, vs, T, d_in, d_out, sem, algo = case
    print(f"random linear_dot case={case}", flush=True)
    A = randn((N, T, d_in), 140 + N + T, 1.0, torch.bfloat16)
    G = randn((N, T, d_out), 141 + d_out, 1e-3, torch.bfloat16)
    semantics = _native.SEM_PAIRWISE_SUM if sem == "pairwise" else _native.SEM_PRESUM
    dot, _ = _native.ops().linear_dot(A.to(gpu), G.to(gpu), n_val, val_start=vs,
                                      semantics=semantics, algo=algo)
    want = R.linear_dot_exact(A, G, n_val, sem, val_start=vs)
    assert_close(dot.cpu(), want, BF16_TOL, f"{sem}/{algo}")


@pytest.mark.parametrize("case", _random_dot_cases(16, 2028))
def test_linear_train_grad_random_shapes(gpu, case):
    """gs_linear_train_grad over seeded random shapes (Linear and Conv1D layouts, bf16 and
    fp32 outputs) against the float64 GEMM; shapes outside the kernel decline with None."""
    N, n_val, vs, T, d_in, d_out, _, algo = case
    conv1d = algo == _native.ALGO_GHOST
    out_dtype = torch.float32 if T % 2 else torch.bfloat16
    print(f"random train grad case={case} conv1d={conv1d} out={out_dtype}", flush=True)
    A = randn((N, T, d_in), 150 + N + T, 1.0, torch.bfloat16)
    G = randn((N, T, d_out), 151 + d_in, 1e-3, torch.bfloat16)
    n_t = N - n_val
    out = _native.ops().linear_train_grad(A.to(gpu), G.to(gpu), n_val, 1.0 / n_t, val_start=vs,
                                          out_dtype=out_dtype, conv1d=conv1d)
    if d_in % 8 or d_out % 8:
        assert out is None
        return
    assert out is not None
    tol = 1e-2 if out_dtype == torch.bfloat16 else FP32_TOL
    assert_close(out.float().cpu(), _train_grad_want(A, G, n_val, vs, 1.0 / n_t, conv1d, gpu),
                 tol, "train grad")
