"""Host-side algebra of the device fit (rfill.ridge) against the oracle, on the CPU: raw sums re-centred
on the reference's shifts give the reference's state; the Cholesky solve gives the eigendecomposition's
maps; residual / combine agree with the oracle's. (The device accumulation is tested in test_gpu_fit.py.)"""
import torch

from oracle import ridge as oridge
from rfill import ridge


def _data(n=3000, d=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, d, generator=g) * torch.linspace(0.5, 2.0, d) + 1.5).to(torch.bfloat16)
    t = torch.eye(d) + 0.2 * torch.randn(d, d, generator=g)
    y = (x.float() @ t + 0.1 * torch.randn(n, d, generator=g)).to(torch.bfloat16)
    return x, {7: y}


def _raw_stats(x, ys, block):
    """rfill.ridge.RidgeStats with its raw device sums filled by exact fp64 math (CPU)."""
    st = ridge.RidgeStats(3, list(ys), x.shape[1], device="cpu")
    xd = x.double()
    st.cx = x[:block].float().mean(0)
    st.s1x += xd.sum(0)
    st.sxx += xd.T @ xd
    for i, y in ys.items():
        st.cy[i] = y[:block].float().mean(0)
        st.s1y[i] += y.double().sum(0)
        st.sxy[i] += xd.T @ y.double()
    st.n = x.shape[0]
    return st.state()


def rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


def test_state_recentres_on_the_first_blocks_means():
    x, ys = _data()
    mine = _raw_stats(x, ys, 1024)
    ref = oridge.RidgeStats(3, [7], 16)
    ref.add(x, ys, block=1024)
    ref = ref.state()
    assert torch.equal(mine["cx"], ref["cx"]) and torch.equal(mine["cy"][7], ref["cy"][7])
    for k in ("sx", "sxx"):
        assert rel(mine[k], ref[k]) < 1e-5, k
    assert rel(mine["sxy"][7], ref["sxy"][7]) < 1e-5 and rel(mine["sy"][7], ref["sy"][7]) < 1e-4
    assert mine["n"] == ref["n"] == 3000


def test_cholesky_solve_equals_eigendecomposition():
    x, ys = _data(seed=1)
    ref = oridge.RidgeStats(3, [7], 16)
    ref.add(x, ys, block=1024)
    st = ref.state()
    ofit = oridge.RidgeFit(st)
    mfit = ridge.RidgeFit(st, device="cpu")
    for lam in (1e-4, 1e-2, 1.0):
        w_ref, b_ref = ofit.layer_f64(7, lam)
        w, b = mfit.layer(7, (lam,))[lam]
        assert rel(w, w_ref) < 1e-6 and rel(b, b_ref) < 1e-6


def test_residual_and_combine_agree_with_the_oracle():
    x, ys = _data(seed=2)
    a, b = oridge.RidgeStats(3, [7], 16), oridge.RidgeStats(3, [7], 16)
    a.add(x[:1500], {7: ys[7][:1500]}, block=512)
    b.add(x[1500:], {7: ys[7][1500:]}, block=512)
    sa, sb = a.state(), b.state()
    mine, ref = ridge.combine(sa, sb, 0.5), oridge.combine(sa, sb, 0.5)
    for k in ("sx", "sxx"):
        assert torch.equal(mine[k], ref[k])
    assert torch.equal(mine["sxy"][7], ref["sxy"][7]) and mine["n"] == ref["n"]
    r1, r2 = ridge.residual(sa), oridge.residual(sa)
    assert torch.equal(r1["sxy"][7], r2["sxy"][7]) and torch.equal(r1["cy"][7], r2["cy"][7])
