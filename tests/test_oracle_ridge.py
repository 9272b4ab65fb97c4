"""Pins the oracle's closed-form ridge and its sufficient statistics by independent computations."""
import numpy as np
import torch

from oracle import ridge


def _data(n=700, d=12, dout=12, seed=0, noise=0.1):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g) * torch.linspace(0.5, 3.0, d) + 2.0
    t = torch.eye(d, dout) + 0.3 * torch.randn(d, dout, generator=g)
    c = torch.randn(dout, generator=g)
    y = x @ t + c + noise * torch.randn(n, dout, generator=g)
    return x, y, t, c


def close(a, b, tol=1e-6):
    """Relative Frobenius agreement: fp32 block products summed in fp64 against an fp64 recomputation."""
    err = float((a.double() - b.double()).norm() / b.double().norm())
    assert err < tol, err


def _stats(x, ys, block=256):
    st = ridge.RidgeStats(3, list(ys), x.shape[1], out_dim=next(iter(ys.values())).shape[1])
    st.add(x, ys, block=block)
    return st.state()


def test_sums_equal_naive_recomputation():
    """Shifted sums == a direct recomputation with the first block's means (code/tests/test_qwen3.py:150-156)."""
    x, y, _, _ = _data()
    s = _stats(x, {5: y}, block=256)
    cx, cy = x[:256].mean(0), y[:256].mean(0)
    xc, yc = (x - cx).double(), (y - cy).double()
    close(s["sxx"], xc.T @ xc)
    close(s["sxy"][5], xc.T @ yc)
    close(s["sx"], xc.sum(0))
    close(s["sy"][5], yc.sum(0))
    assert s["n"] == 700


def test_ridge_equals_augmented_least_squares():
    """W(lam) = argmin |Xc W - Yc|^2 + lam s |W|^2, s = mean diag of the centred scatter, bias
    unpenalised, solved independently as least squares on [Xc; sqrt(lam s) I]."""
    x, y, _, _ = _data()
    fit = ridge.RidgeFit(_stats(x, {5: y}))
    xd, yd = x.double().numpy(), y.double().numpy()
    mx, my = xd.mean(0), yd.mean(0)
    xc, yc = xd - mx, yd - my
    s = np.mean(np.diag(xc.T @ xc))
    for lam in (1e-4, 1e-2, 1.0):
        aug_x = np.vstack([xc, np.sqrt(lam * s) * np.eye(x.shape[1])])
        aug_y = np.vstack([yc, np.zeros((x.shape[1], y.shape[1]))])
        w = np.linalg.lstsq(aug_x, aug_y, rcond=None)[0]
        weight, bias = fit.layer(5, (lam,))[lam]
        np.testing.assert_allclose(weight.double().numpy(), w.T, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(bias.double().numpy(), my - mx @ w, rtol=1e-4, atol=1e-5)


def test_small_lambda_is_ols_and_recovers_a_noiseless_map():
    x, y, t, c = _data(noise=0.0)
    fit = ridge.RidgeFit(_stats(x, {5: y}))
    weight, bias = fit.layer_f64(5, 1e-12)
    torch.testing.assert_close(weight, t.T.double(), atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(bias, c.double(), atol=1e-6, rtol=1e-6)
    xn, yn, _, _ = _data(noise=0.3, seed=2)
    fit = ridge.RidgeFit(_stats(xn, {5: yn}))
    ols = np.linalg.lstsq(np.hstack([xn.double().numpy(), np.ones((700, 1))]), yn.double().numpy(), rcond=None)[0]
    weight, bias = fit.layer_f64(5, 1e-12)
    np.testing.assert_allclose(weight.numpy(), ols[:-1].T, atol=2e-6)   # fp32 block products in the sums
    np.testing.assert_allclose(bias.numpy(), ols[-1], atol=2e-6)


def test_lambda_shrinks_towards_zero():
    x, y, _, _ = _data()
    fit = ridge.RidgeFit(_stats(x, {5: y}))
    norms = [fit.layer_f64(5, lam)[0].norm().item() for lam in (1e-3, 1e-1, 10.0, 1e3)]
    assert all(a > b for a, b in zip(norms, norms[1:]))


def test_combine_equals_concatenation():
    """combine(a, b, 1) == the sums over both row sets (code/kva/ridge.py:142-156)."""
    x, y, _, _ = _data(n=900)
    a, b = _stats(x[:500], {5: y[:500]}), _stats(x[500:], {5: y[500:]})
    both = ridge.combine(a, b, 1.0)
    cx, cy = a["cx"], a["cy"][5]
    xc, yc = x.double() - cx, y.double() - cy
    close(both["sxx"], xc.T @ xc)
    close(both["sxy"][5], xc.T @ yc)
    close(both["sy"][5], yc.sum(0))
    assert both["n"] == 900


def test_residual_is_the_fit_of_y_minus_x():
    """residual(state) holds the statistics of y - x: its OLS map is the direct map minus I."""
    x, y, _, _ = _data()
    st = _stats(x, {5: y})
    w_direct, b_direct = ridge.RidgeFit(st).layer_f64(5, 1e-12)
    w_res, b_res = ridge.RidgeFit(ridge.residual(st)).layer_f64(5, 1e-12)
    torch.testing.assert_close(w_res + torch.eye(12, dtype=torch.float64), w_direct, atol=1e-8, rtol=1e-8)
    torch.testing.assert_close(b_res, b_direct, atol=1e-8, rtol=1e-8)


def test_capture_shift_is_the_first_documents_mean():
    """fit_sweep's capture: shifts are the first document's means; sums over every document
    (code/scripts/fit_sweep.py:94-111)."""
    g = torch.Generator().manual_seed(4)
    docs = [{2: torch.randn(n, 6, generator=g) + 1, 3: torch.randn(n, 6, generator=g) - 1} for n in (30, 50)]
    cap = ridge.Capture([2], 4, 6)
    for d in docs:
        cap.add_document(d)
    cx, cy = docs[0][2].mean(0), docs[0][3].mean(0)
    xc = torch.cat([d[2] for d in docs]) - cx
    yc = torch.cat([d[3] for d in docs]) - cy
    s = cap.state(2)
    close(s["sxx"], xc.double().T @ xc.double())
    close(s["sxy"][3], xc.double().T @ yc.double())
    assert s["n"] == 80 and s["layers"] == [2, 3]
