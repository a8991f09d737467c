"""gs_linear_dot_noalloc (the allocation-free variant of gs_linear_dot) through the C ABI
against gs_linear_dot on the same inputs: the same plan and kernels, so the outputs are
bit-identical.  Two calls in a row on the shared scratch array, the second with a smaller
input, for each case."""
import pytest
import torch

from ghostsuite_amd import _native
from tests.helpers import randn

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16

# (N, n_val, T, d_in, d_out, dtype, semantics, algo, pairs): a large call, then a smaller one
CASES = [
    ((20, 4, 1024, 768, 3072, BF16, _native.SEM_PAIRWISE_SUM, _native.ALGO_AUTO, False),
     (6, 2, 256, 256, 512, BF16, _native.SEM_PAIRWISE_SUM, _native.ALGO_AUTO, False)),
    ((20, 4, 1024, 768, 2304, BF16, _native.SEM_PRESUM, _native.ALGO_AUTO, False),
     (7, 3, 300, 200, 136, BF16, _native.SEM_PRESUM, _native.ALGO_VALGRAD, False)),
    ((32, 8, 512, 768, 3072, BF16, _native.SEM_PAIRWISE_SUM, _native.ALGO_GHOST, False),
     (10, 3, 64, 128, 96, BF16, _native.SEM_PAIRWISE_SUM, _native.ALGO_GHOST, True)),
    ((12, 4, 130, 64, 40, torch.float32, _native.SEM_PAIRWISE_SUM, _native.ALGO_VALGRAD, True),
     (6, 2, 5, 24, 40, torch.float32, _native.SEM_PRESUM, _native.ALGO_GHOST, False)),
]


def _inputs(case, seed, dev):
    N, n_val, T, d_in, d_out, dt, sem, algo, pairs = case
    A = randn((N, T, d_in), seed, 1.0, dt).to(dev)
    G = randn((N, T, d_out), seed + 1, 1e-3, dt).to(dev)
    return A, G


@pytest.mark.parametrize("big,small", CASES)
def test_noalloc_matches_workspace_entry_point(gpu, big, small):
    ops = _native.ops()
    for k, case in enumerate((big, small)):
        N, n_val, T, d_in, d_out, dt, sem, algo, pairs = case
        print(f"noalloc case={case[:5]} {dt} sem={sem} algo={algo} pairs={pairs}", flush=True)
        A, G = _inputs(case, 900 + 10 * k + T, gpu)
        vs = 1 if k == 0 else N - n_val
        want, want_pair = ops.linear_dot(A, G, n_val, val_start=vs, semantics=sem, algo=algo,
                                         want_pair=pairs)
        out = torch.full((N - n_val,), float("nan"), device=gpu)
        pair = torch.full((n_val, N - n_val), float("nan"), device=gpu) if pairs else None
        ops.linear_dot_noalloc(A, G, n_val, out, pair, val_start=vs, semantics=sem, algo=algo)
        torch.cuda.synchronize()
        assert torch.equal(out, want), (out[:4], want[:4])
        if pairs:
            assert torch.equal(pair, want_pair)
