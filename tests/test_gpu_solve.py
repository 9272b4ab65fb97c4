"""GPU parity of the ridge solve (rf_ridge_solve: the inverse of C + lam s I by block recursion on Schur
complements over a 64 x 64 Gauss-Jordan base, fp64 MFMA products) against torch.linalg.solve in fp64 on the
same device (the checker), for sizes on and off the 64-multiple grid (the padded identity block), several
right-hand-side widths and lambdas, and the bias mean_y - mean_x W. Bar: 1e-10 relative Frobenius (fp64
arithmetic on matrices of condition number up to ~1e4)."""
import pytest
import torch

pytestmark = pytest.mark.gpu
TOL = 1e-10


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _spd(d, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(4 * d, d, generator=g, device=dev, dtype=torch.float64)
    x[:, :3] *= 20                                        # outlier channels, as in the fit workload
    xc = x - x.mean(0)
    return xc.T @ xc, g


def rel(a, b):
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("d,R", [(64, 64), (100, 2), (192, 200), (512, 1024), (1000, 130), (4096, 256)])
def test_ridge_solve_matches_fp64_solve(dev, d, R):
    from rfill.ridge import RidgeFit
    C, g = _spd(d, d, dev)
    B = torch.randn(d, R, generator=g, device=dev, dtype=torch.float64) * 50
    fit = RidgeFit.__new__(RidgeFit)
    fit.device, fit.cxx = dev, C.contiguous()
    fit.scale = C.diagonal().mean().item()
    fit.mean_x = torch.randn(d, generator=g, device=dev, dtype=torch.float64)
    mean_y = torch.randn(R, generator=g, device=dev, dtype=torch.float64)
    lams = (1e-4, 1e-2, 1.0)
    w, b = fit.solve(B, lams, mean_y)
    torch.cuda.synchronize()
    worst = 0.0
    for li, lam in enumerate(lams):
        want = torch.linalg.solve(C + lam * fit.scale * torch.eye(d, device=dev, dtype=torch.float64), B)
        worst = max(worst, rel(w[li], want), rel(b[li], mean_y - fit.mean_x @ want))
    print(f"rf_ridge_solve d {d}, R {R}: worst rel err {worst:.2e}")
    assert worst < TOL


def test_ridge_solve_refuses(dev):
    from rfill.ridge import RidgeFit
    C, g = _spd(64, 1, dev)
    fit = RidgeFit.__new__(RidgeFit)
    fit.device, fit.cxx, fit.scale = dev, C.contiguous(), C.diagonal().mean().item()
    fit.mean_x = torch.zeros(64, device=dev, dtype=torch.float64)
    with pytest.raises(ValueError, match="positive"):
        fit.solve(torch.ones(64, 2, device=dev, dtype=torch.float64), (0.0,))
    with pytest.raises(ValueError, match="even"):
        fit.solve(torch.ones(64, 3, device=dev, dtype=torch.float64), (1.0,))
