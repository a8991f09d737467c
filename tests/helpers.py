"""Shared test utilities (seeded inputs, tolerance checks)."""
import torch

from oracle.ghost_ref import normwise_close

BF16_TOL = 2e-2     # north-star bf16 tolerance, normwise
FP32_TOL = 1e-4     # north-star fp32 tolerance, normwise


def gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, seed, scale=1.0, dtype=torch.float32):
    return (torch.randn(shape, generator=gen(seed), dtype=torch.float32) * scale).to(dtype)


def assert_close(x, y, tol, what=""):
    ok, worst = normwise_close(x, y, tol)
    assert ok, f"{what}: worst normwise error {worst:.3e} > {tol:.1e}\n got {x.reshape(-1)[:6]}\n want {y.reshape(-1)[:6]}"
    return worst
