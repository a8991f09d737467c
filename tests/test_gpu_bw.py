"""GPU parity of the Embedding, LayerNorm and Kronecker-projection kernels (C ABI)."""
import pytest
import torch

from ghostsuite_amd import _native
from oracle import ghost_ref as R
from tests.helpers import BF16_TOL, FP32_TOL, assert_close, gen, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(6, 2, 5, 24, 11), (20, 4, 64, 96, 50), (10, 3, 33, 40, 3000)])
def test_embedding_dot(gpu, dtype, shape):
    N, n_val, T, d, vocab = shape
    ids = torch.randint(0, vocab, (N, T), generator=gen(3 + T))
    G = randn((N, T, d), 4 + T, 1e-3, dtype)
    for val_start in (N - n_val, 0):
        print(f"embedding shape={shape} dtype={dtype} val_start={val_start}", flush=True)
        dot = _native.ops().embedding_dot(ids.to(gpu), G.to(gpu), n_val, vocab,
                                          val_start=val_start)
        torch.cuda.synchronize()
        want = R.embedding_dot_exact(ids, G, n_val, val_start=val_start)
        tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
        assert_close(dot.cpu(), want, tol, "embedding dot")


@pytest.mark.parametrize("shape", [(20, 4, 1024, 64, 50257), (5, 2, 4096, 24, 1000),
                                   (6, 3, 1500, 40, 2)])
def test_embedding_dot_sort_sizes(gpu, shape):
    """The sorted-segment path at full size: 4096 val keys (the GPT-2 wte batch), the 8192-key
    maximum with runs of ~8 equal ids, and 4500 keys in two long runs."""
    N, n_val, T, d, vocab = shape
    ids = torch.randint(0, vocab, (N, T), generator=gen(41 + T))
    G = randn((N, T, d), 42 + T, 1e-3, torch.bfloat16)
    print(f"embedding sort shape={shape}", flush=True)
    dot = _native.ops().embedding_dot(ids.to(gpu), G.to(gpu), n_val, vocab)
    torch.cuda.synchronize()
    assert_close(dot.cpu(), R.embedding_dot_exact(ids, G, n_val), BF16_TOL, "embedding dot")


@pytest.mark.parametrize("shape", [(8, 2, 300, 24, 50), (20, 4, 1024, 16, 50257)])
def test_embedding_dot_out_of_range_ids(gpu, shape):
    """Ids outside [0, vocab) (negative or too large) take no part, as val or train tokens:
    the dot equals the closed form with those tokens' gradient rows zeroed."""
    N, n_val, T, d, vocab = shape
    ids = torch.randint(0, vocab, (N, T), generator=gen(51 + T))
    bad = torch.rand(N, T, generator=gen(52 + T)) < 0.1
    ids[bad] = torch.where(torch.rand(N, T, generator=gen(53 + T)) < 0.5,
                           torch.full((N, T), -3), torch.full((N, T), vocab + 7))[bad]
    G = randn((N, T, d), 54 + T, 1e-3, torch.bfloat16)
    print(f"embedding out-of-range ids shape={shape}", flush=True)
    dot = _native.ops().embedding_dot(ids.to(gpu), G.to(gpu), n_val, vocab)
    torch.cuda.synchronize()
    Gz = G.clone()
    Gz[bad] = 0
    assert_close(dot.cpu(), R.embedding_dot_exact(ids.clamp(0, vocab - 1), Gz, n_val), BF16_TOL,
                 "embedding dot")


@pytest.mark.parametrize("shape", [(6, 3, 3000, 16, 100), (5, 2, 40, 24, 600_000)])
def test_embedding_dot_fixed_point_path(gpu, shape):
    """More than 8192 val tokens, or ids of 2^19 and above: the fixed-point segment path."""
    N, n_val, T, d, vocab = shape
    ids = torch.randint(0, vocab, (N, T), generator=gen(31 + T))
    G = randn((N, T, d), 32 + T, 1e-3, torch.bfloat16)
    print(f"embedding fixed-point shape={shape}", flush=True)
    dot = _native.ops().embedding_dot(ids.to(gpu), G.to(gpu), n_val, vocab)
    torch.cuda.synchronize()
    assert_close(dot.cpu(), R.embedding_dot_exact(ids, G, n_val), BF16_TOL, "embedding dot")


def test_embedding_positions_and_all_equal_ids(gpu):
    N, n_val, T, d = 8, 2, 40, 32
    G = randn((N, T, d), 9, 1e-3)
    pos = torch.arange(T).repeat(N, 1)   # per-sample position ids (wpe)
    dot = _native.ops().embedding_dot(pos.to(gpu), G.to(gpu), n_val, T)
    same = torch.full((N, T), 7)
    dot2 = _native.ops().embedding_dot(same.to(gpu), G.to(gpu), n_val, 50)
    torch.cuda.synchronize()
    # positions: dot_i = sum_t <g_it, sum_j g_jt>
    tr, va = G[:N - n_val].double(), G[N - n_val:].double()
    assert_close(dot.cpu(), (tr * va.sum(0)).sum((1, 2)), FP32_TOL, "positions")
    # one shared id: dot_i = <sum_t g_it, sum_{j,s} g_js>
    assert_close(dot2.cpu(), tr.sum(1) @ va.sum((0, 1)), FP32_TOL, "all-equal ids")


def _emb_grad_exact(ids, G, n_val, vs, vocab, scale):
    N, d = G.shape[0], G.shape[-1]
    tr_i, _ = R.split_rows(ids.reshape(N, -1).long(), n_val, vs)
    tr_g, _ = R.split_rows(G.double().reshape(N, -1, d), n_val, vs)
    keep = (tr_i >= 0) & (tr_i < vocab)
    g = torch.zeros(vocab, d, dtype=torch.float64)
    g.index_add_(0, tr_i[keep], tr_g[keep])
    touched = torch.zeros(vocab, dtype=torch.bool)
    touched[tr_i[keep]] = True
    return g * scale, touched


@pytest.mark.parametrize("gdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [
    # N, n_val, T, d, vocab
    (6, 2, 5, 24, 11),            # many tokens per id
    (20, 4, 1024, 768, 50257),    # GPT-2 wte: 16 train rows of 1024 tokens
    (10, 2, 2048, 2048, 50304),   # Pythia wte
    (7, 3, 33, 20, 3000),         # d not a multiple of 8: scalar loads
    (5, 1, 1024, 64, 1),          # every token the same id: one 4096-token segment
])
def test_embedding_train_grad(gpu, gdt, odt, shape):
    """gs_embedding_train_grad against float64 index_add of the train rows: overwrite mode
    (every row written, zeros where no train token has the id) and accumulate mode (only the
    touched rows change), val block in the middle, out-of-range ids skipped, bit-identical on
    a second run."""
    N, n_val, T, d, vocab = shape
    ids = torch.randint(0, vocab, (N, T), generator=gen(80 + T))
    ids[0, :3] = -1
    ids[-1, -2:] = vocab + 5
    G = randn((N, T, d), 81 + T, 1e-2, gdt)
    vs = 1 if N - n_val > 1 else 0
    scale = N / (N - n_val)
    print(f"embedding train grad shape={shape} G {gdt} out {odt}", flush=True)
    idd, Gd = ids.to(gpu), G.to(gpu)
    out = torch.full((vocab, d), float("nan"), dtype=odt, device=gpu)
    _native.ops().embedding_train_grad(idd, Gd, n_val, scale, out, val_start=vs)
    want, touched = _emb_grad_exact(ids, G, n_val, vs, vocab, scale)
    tol = 1e-2 if odt == torch.bfloat16 else FP32_TOL
    got = out.cpu()
    assert_close(got, want, tol, "overwrite")
    assert torch.all(got[~touched] == 0)
    again = torch.empty_like(out)
    _native.ops().embedding_train_grad(idd, Gd, n_val, scale, again, val_start=vs)
    assert torch.equal(again, out)
    prev = randn((vocab, d), 82, 1e-2, odt)
    acc = prev.to(gpu)
    _native.ops().embedding_train_grad(idd, Gd, n_val, scale, acc, accumulate=True, val_start=vs)
    got = acc.cpu()
    assert torch.equal(got[~touched], prev[~touched])
    assert_close(got, prev.double() + want, tol, "accumulate")


@pytest.mark.parametrize("shape,pad_frac", [
    # N, n_val, T, d, vocab
    ((34, 2, 2048, 256, 50257), 0.9),   # 65536 train tokens, 90% one pad id
    ((9, 1, 1000, 72, 40), 0.0),        # runs of ~200 tokens across many windows
    ((3, 1, 4099, 8, 50257), 1.0),      # every train token the pad id, ragged T
    ((5, 1, 900, 16, 2_000_000), 0.3),  # ids of 2^20 and above: 64-bit sort keys
    ((4, 1, 3000, 10, 7), 0.97),        # long runs, rows of 10 features (no whole float4s)
    ((40, 2, 2048, 768, 50257), 0.9),   # GPT-2 width: a 70k-token run over many workgroups
])
def test_embedding_train_grad_heavy_ids(gpu, shape, pad_frac):
    """Ids that repeat thousands of times (a padded batch): the sorted-list pipeline stays
    linear in the token count (the call is timed against a generous bound) and sums each
    run in a fixed order (bit-identical on a second run), against float64 index_add.  A run
    longer than a few hundred tokens is summed by the workgroups whose windows it covers,
    each taking feature slices; shorter ones by the workgroup where they begin."""
    import time
    N, n_val, T, d, vocab = shape
    ids = torch.randint(0, vocab, (N, T), generator=gen(90 + T))
    pad = torch.rand(N, T, generator=gen(91 + T)) < pad_frac
    ids[pad] = vocab - 1
    G = randn((N, T, d), 92 + T, 1e-2, torch.bfloat16)
    scale = N / (N - n_val)
    print(f"embedding train grad heavy ids shape={shape} pad={pad_frac}", flush=True)
    idd, Gd = ids.to(gpu), G.to(gpu)
    out = torch.empty((vocab, d), dtype=torch.float32, device=gpu)
    ops = _native.ops()
    ops.embedding_train_grad(idd, Gd, n_val, scale, out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    again = torch.empty_like(out)
    ops.embedding_train_grad(idd, Gd, n_val, scale, again)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"  one call {dt * 1e3:.2f} ms", flush=True)
    assert dt < 0.05, f"{dt * 1e3:.1f} ms for {(N - n_val) * T} tokens"
    assert torch.equal(again, out)
    want, touched = _emb_grad_exact(ids, G, n_val, N - n_val, vocab, scale)
    got = out.cpu()
    assert_close(got, want, FP32_TOL, "heavy ids")
    assert torch.all(got[~touched] == 0)
    prev = randn((vocab, d), 93, 1e-2, torch.bfloat16)
    acc = prev.to(gpu)
    ops.embedding_train_grad(idd, Gd, n_val, scale, acc, accumulate=True)
    got = acc.cpu()
    assert torch.equal(got[~touched], prev[~touched])
    assert_close(got, prev.double() + want, 1e-2, "heavy ids, accumulate")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(6, 2, 5, 24), (20, 4, 70, 768), (5, 1, 3, 2048), (4, 1, 2, 100),
                                   (3, 1, 130, 1024), (4, 2, 64, 1600), (20, 4, 1024, 768),
                                   (10, 2, 2048, 2048), (5, 2, 9, 6),
                                   # wider than the register-resident kernels: row statistics
                                   # first, then the feature pass
                                   (3, 1, 70, 2560), (4, 2, 33, 4100), (2, 1, 130, 8192),
                                   (3, 1, 5, 2049)])
@pytest.mark.parametrize("mid", [False, True])
def test_layernorm_dots_and_grads(gpu, dtype, shape, mid):
    """LayerNorm dots and grads against float64; `mid`: the val block between train rows
    (the oracle sees the same samples with the val block moved to the end)."""
    N, n_val, T, Fd = shape
    X = randn((N, T, Fd), 11 + T, 2.0, dtype) + 0.5
    G = randn((N, T, Fd), 12 + T, 1e-3, dtype)
    n_t = N - n_val
    vs = 1 if mid else N - n_val
    print(f"layernorm shape={shape} dtype={dtype} val_start={vs}", flush=True)
    dw, db, gw, gb = _native.ops().layernorm_dot(X.to(gpu), G.to(gpu), n_val, 1e-5, val_start=vs,
                                                 grad_scale=N / n_t, grad_dtype=torch.float32)
    torch.cuda.synchronize()
    X = torch.cat([X[:vs], X[vs + n_val:], X[vs:vs + n_val]])  # val rows last
    G = torch.cat([G[:vs], G[vs + n_val:], G[vs:vs + n_val]])
    ww, wb = R.layernorm_dot_exact(X, G, n_val, 1e-5)
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert_close(dw.cpu(), ww, tol, "ln weight dot")
    assert_close(db.cpu(), wb, tol, "ln bias dot")
    gw_ref, gb_ref = R.layernorm_train_grad(X.double(), G.double() * N, n_val, 1e-5)
    assert_close(gw.cpu(), gw_ref, tol, "ln weight grad")
    assert_close(gb.cpu(), gb_ref, tol, "ln bias grad")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("conf", [
    # B, T, n_i, n_o, k_i, k_o
    (3, 5, 24, 40, 4, 6),
    (4, 130, 256, 512, 16, 16),
    (2, 64, 96, 384, 28, 9),
    (2, 3, 1, 10, 1, 8),
    # the reference's own rank settings (choose_ki_ko, projection_utils.py:12-66):
    (3, 100, 768, 3072, 43, 12),     # fc at rank 512, k_min 8
    (3, 100, 3072, 768, 11, 47),     # fc_out at rank 512
    (2, 70, 1024, 4096, 64, 16),     # fc at rank 1024 (64-row slice boundary)
    (2, 70, 1024, 50257, 157, 8),    # lm_head at rank 512: three 64-row slices of P_i
    (2, 33, 200, 300, 70, 130),      # more than 64 rows on both sides
])
@pytest.mark.parametrize("conv1d", [False, True])
def test_kron_projection(gpu, dtype, conf, conv1d):
    B, T, n_i, n_o, k_i, k_o = conf
    A = randn((B, T, n_i), 21 + T, 1.0, dtype)
    G = randn((B, T, n_o), 22 + T, 1e-3, dtype)
    if conv1d:   # Conv1D: P_i acts on the output grads (width n_o), P_o on the inputs
        P_i = randn((k_i, n_o), 23, 1.0 / k_i ** 0.5)
        P_o = randn((k_o, n_i), 24, 1.0 / k_o ** 0.5)
        layout = _native.PROJ_KI_KO
    else:
        P_i = randn((k_i, n_i), 23, 1.0 / k_i ** 0.5)
        P_o = randn((k_o, n_o), 24, 1.0 / k_o ** 0.5)
        layout = _native.PROJ_KO_KI
    print(f"kron conf={conf} dtype={dtype} conv1d={conv1d}", flush=True)
    out = _native.ops().kron_proj(A.to(gpu), G.to(gpu), P_i.to(gpu), P_o.to(gpu), float(B),
                                  layout=layout)
    torch.cuda.synchronize()
    want = R.kron_proj_exact(A.float(), G.float(), P_i.to(dtype).float(), P_o.to(dtype).float(),
                             float(B), conv1d=conv1d)
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert_close(out.cpu(), want, tol, "kron")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("conf", [
    # B, T, vocab, d, k_i, k_o
    (3, 5, 30, 24, 4, 6),
    (4, 130, 50257, 768, 16, 16),    # GPT-2 vocabulary, two token chunks + a tail
    (2, 64, 1000, 100, 32, 32),      # d not a multiple of 8: scalar G loads
    (5, 1, 7, 8, 1, 3),
    (3, 130, 50257, 768, 4, 64),     # wte at the reference's default rank 256, k_min 4
    (2, 70, 50257, 1024, 8, 128),    # wte at rank 1024: two 64-row slices of P_o
    (2, 40, 3000, 96, 100, 5),       # gathered side wider than 64 columns
])
def test_kron_embedding_projection(gpu, dtype, conf):
    B, T, V, d, k_i, k_o = conf
    ids = torch.randint(0, V, (B, T), generator=gen(31 + T))
    ids[0, : min(T, 3)] = ids[0, 0]               # repeated ids in one sample
    G = randn((B, T, d), 32 + T, 1e-3, dtype)
    P_i = randn((k_i, V), 33, 1.0 / k_i ** 0.5)
    P_o = randn((k_o, d), 34, 1.0 / k_o ** 0.5)
    print(f"kron_embed conf={conf} dtype={dtype}", flush=True)
    out = _native.ops().kron_embed_proj(ids.to(gpu), G.to(gpu), P_i.t().contiguous().to(gpu),
                                        P_o.to(gpu), 1.0)
    torch.cuda.synchronize()
    want = R.kron_embed_proj_exact(ids, G.float(), P_i.to(dtype).float(), P_o.to(dtype).float())
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert_close(out.cpu(), want, tol, "kron embed")


def _random_bw_cases(n, seed):
    """Seeded (N, n_val, val_start, T, d, vocab) for the bandwidth ops: any T and feature
    count (aligned or not), small to 50k vocabularies, 1-4 val rows anywhere, at least four
    train rows."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    out = []
    for _ in range(n):
        n_val = pick(1, 4)
        N = n_val + pick(4, 8)
        d = 8 * pick(1, 200) if pick(0, 1) else pick(1, 1500)
        vocab = [pick(1, 40), pick(100, 5000), 50257][pick(0, 2)]
        out.append((N, n_val, pick(0, N - n_val), pick(1, 300), d, vocab))
    return out


@pytest.mark.parametrize("case", _random_bw_cases(16, 2029))
def test_layernorm_random_shapes(gpu, case):
    """LayerNorm dots and train gradients over seeded random shapes against float64."""
    N, n_val, vs, T, Fd, _ = case
    print(f"random layernorm case={case}", flush=True)
    X = randn((N, T, Fd), 160 + T, 2.0, torch.bfloat16) + 0.5
    G = randn((N, T, Fd), 161 + Fd, 1e-3, torch.bfloat16)
    n_t = N - n_val
    dw, db, gw, gb = _native.ops().layernorm_dot(X.to(gpu), G.to(gpu), n_val, 1e-5, val_start=vs,
                                                 grad_scale=N / n_t, grad_dtype=torch.float32)
    X = torch.cat([X[:vs], X[vs + n_val:], X[vs:vs + n_val]])  # val rows last for the oracle
    G = torch.cat([G[:vs], G[vs + n_val:], G[vs:vs + n_val]])
    ww, wb = R.layernorm_dot_exact(X, G, n_val, 1e-5)
    assert_close(dw.cpu(), ww, BF16_TOL, "ln weight dot")
    assert_close(db.cpu(), wb, BF16_TOL, "ln bias dot")
    gw_ref, gb_ref = R.layernorm_train_grad(X.double(), G.double() * N, n_val, 1e-5)
    assert_close(gw.cpu(), gw_ref, BF16_TOL, "ln weight grad")
    assert_close(gb.cpu(), gb_ref, BF16_TOL, "ln bias grad")


@pytest.mark.parametrize("case", _random_bw_cases(16, 2030))
def test_embedding_random_shapes(gpu, case):
    """Embedding dot and train gradient over seeded random shapes and vocabularies (a few ids
    out of range) against float64."""
    N, n_val, vs, T, d, vocab = case
    print(f"random embedding case={case}", flush=True)
    ids = torch.randint(0, vocab, (N, T), generator=gen(170 + T))
    ids[0, 0] = -1
    G = randn((N, T, d), 171 + d, 1e-3, torch.bfloat16)
    idd, Gd = ids.to(gpu), G.to(gpu)
    dot = _native.ops().embedding_dot(idd, Gd, n_val, vocab, val_start=vs)
    want = R.embedding_dot_exact(ids.clamp(0, vocab - 1), G * (ids >= 0).unsqueeze(-1), n_val,
                                 val_start=vs)
    assert_close(dot.cpu(), want, BF16_TOL, "embedding dot")
    scale = N / (N - n_val)
    out = torch.full((vocab, d), float("nan"), dtype=torch.float32, device=gpu)
    _native.ops().embedding_train_grad(idd, Gd, n_val, scale, out, val_start=vs)
    g_want, touched = _emb_grad_exact(ids, G, n_val, vs, vocab, scale)
    got = out.cpu()
    assert_close(got, g_want, FP32_TOL, "embedding train grad")
    assert torch.all(got[~touched] == 0)


@pytest.mark.parametrize("case", _random_bw_cases(12, 2031))
def test_kron_projection_random_shapes(gpu, case):
    """Kronecker projection (Linear layout) over seeded random shapes and ranks (1-80 rows of
    P on each side) against float64."""
    B, _, _, T, n_i, n_o = case
    g = torch.Generator().manual_seed(B * 1000 + T)
    k_i, k_o = int(torch.randint(1, 81, (1,), generator=g)), int(torch.randint(1, 81, (1,), generator=g))
    n_o = max(1, n_o % 2048)
    print(f"random kron case={(B, T, n_i, n_o, k_i, k_o)}", flush=True)
    A = randn((B, T, n_i), 180 + T, 1.0, torch.bfloat16)
    G = randn((B, T, n_o), 181 + T, 1e-3, torch.bfloat16)
    P_i = randn((k_i, n_i), 182, 1.0 / k_i ** 0.5)
    P_o = randn((k_o, n_o), 183, 1.0 / k_o ** 0.5)
    out = _native.ops().kron_proj(A.to(gpu), G.to(gpu), P_i.to(gpu), P_o.to(gpu), float(B),
                                  layout=_native.PROJ_KO_KI)
    want = R.kron_proj_exact(A.float(), G.float(), P_i.to(torch.bfloat16).float(),
                             P_o.to(torch.bfloat16).float(), float(B))
    assert_close(out.cpu(), want, BF16_TOL, "kron")
