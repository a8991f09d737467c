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


def assert_close_to_sum(got, want, mag, tol, what=""):
    """|got - want| <= tol * max(mag, rms(want)) elementwise, mag = the summed magnitudes of
    the addends of a sum formed from separately rounded contributions (a tied weight's two
    train gradients): the rounding bound of such a sum, which where the addends cancel is
    relative to them, not to the small sum."""
    got = got.double().cpu()
    want = want.double().cpu()
    mag = mag.double().cpu()
    rms = want.pow(2).mean().sqrt().item()
    worst = ((got - want).abs() / torch.clamp(mag, min=max(rms, 1e-300))).max().item()
    assert worst <= tol, f"{what}: worst error {worst:.3e} of the addends' size > {tol:.1e}"
    return worst


def conv_net():
    """Two Conv2d layers (stride, padding, dilation, rectangular kernels) and a Linear head."""
    from torch import nn
    return nn.Sequential(
        nn.Conv2d(3, 6, kernel_size=3, padding=1, stride=2), nn.ReLU(),
        nn.Conv2d(6, 4, kernel_size=(3, 2), dilation=(1, 2), padding=(1, 0)), nn.ReLU(),
        nn.Flatten(), nn.Linear(4 * 4 * 2, 5))


def conv_net_square():
    """A Conv2d with C_in*kh*kw == C_out whose switch picks the ghost branch (2 L^2 <=
    weight.numel(): L = 16, 36 x 36 weight), then a 1x1 Conv2d on the materialised branch and a
    Linear head, for 8 x 8 inputs with 4 channels."""
    from torch import nn
    return nn.Sequential(
        nn.Conv2d(4, 36, kernel_size=3, padding=1, stride=2), nn.ReLU(),
        nn.Conv2d(36, 4, kernel_size=1), nn.ReLU(),
        nn.Flatten(), nn.Linear(4 * 4 * 4, 5))


def run_conv_engine(model, X, Y, n_val, device, precision="fp32", **options):
    """One GradDotProd step on `model`; returns ({name: dot}, {name: grad}) on the CPU."""
    import torch.nn.functional as F
    from ghostsuite_amd import GradDotProdEngine
    eng = GradDotProdEngine(model, val_batch_size=n_val, use_dummy_bias=False,
                            precision=precision, **options)
    eng.attach(torch.optim.SGD(model.parameters(), lr=0.0))
    eng.attach_train_batch(X[:-n_val], Y[:-n_val], 0, 0)
    F.cross_entropy(model(X.to(device)), Y.to(device)).backward()
    dots = {n: p.grad_dot_prod.detach().cpu().clone() for n, p in model.named_parameters()
            if hasattr(p, "grad_dot_prod")}
    eng.prepare_gradients()
    grads = {n: p.grad.detach().cpu().clone() for n, p in model.named_parameters()}
    eng.aggregate_and_log()
    eng.detach()
    return dots, grads
