"""Host-side algebra of the device fit (rfill.ridge) against the oracle, on the CPU: the device path's sums
emulated exactly in fp64 (the centring chosen from the first block, the centred channels' exact bf16 hi / lo
operand rows, the augmented Gram products), combined and moved onto the reference's shifts by state(), give
the reference's state -- with centring on and off, and when a saved state is resumed; residual / combine agree
with the oracle's. (The device accumulation and the solve, rf_ridge_solve, are tested on the GPU in
test_gpu_fit.py and test_gpu_fit_c5.py.)"""
import torch

from oracle import ridge as oridge
from rfill import ridge


def _data(n=3000, d=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, d, generator=g) * torch.linspace(0.5, 2.0, d) + 1.5).to(torch.bfloat16)
    t = torch.eye(d) + 0.2 * torch.randn(d, d, generator=g)
    y = (x.float() @ t + 0.1 * torch.randn(n, d, generator=g)).to(torch.bfloat16)
    return x, {7: y}


def _centring(rows, c=None, cap=ridge.SHIFT_MAX):
    xd = rows.double()
    return ridge.Centring(xd.sum(0), (xd * xd).sum(0), rows.shape[0], c, cap)


def _operand(x, cen):
    """The transposed operand the device builds, as [rows, cols + lo_rows] fp64: d = x - shift (fp32) as bf16 hi,
    and the centred channels' exact remainder as bf16 mid and lo parts in their extra rows; and the sums of d."""
    d = x.float() - cen.shift
    hi = d.to(torch.bfloat16)
    r1 = d - hi.float()
    mid = r1.to(torch.bfloat16)
    lo = (r1 - mid.float()).to(torch.bfloat16)
    extra = torch.zeros(x.shape[0], cen.lo_rows, dtype=torch.float64)
    extra[:, :cen.s] = mid[:, cen.idx].double()
    extra[:, cen.s:2 * cen.s] = lo[:, cen.idx].double()
    hi = torch.where(cen.lo_row >= 0, hi.float(), x.float()).double()
    return torch.cat((hi, extra), 1), d.double().sum(0)


def _emulate(st, x, ys, block):
    """st (rfill.ridge.RidgeStats on the CPU) with its device sums filled by exact fp64 math."""
    d, o = st.dim, st.out_dim
    if st.cen_x is None:
        b = st.base
        st.cen_x = _centring(x[:block], None if b is None else b["cx"], st.centre_max)
        for i in st.layers:
            st.cen_y[i] = _centring(ys[i][:block], None if b is None else b["cy"][i], st.centre_max)
        f64 = dict(dtype=torch.float64)
        st.sxx = torch.zeros(d + 2 * st.cen_x.s, d + st.cen_x.lo_rows, **f64)
        st.sxy = {i: torch.zeros(d + 2 * st.cen_x.s, o + st.cen_y[i].lo_rows, **f64) for i in st.layers}
    ax, s1 = _operand(x, st.cen_x)
    st.s1x += s1
    st.sxx += ax[:, :d + 2 * st.cen_x.s].T @ ax[:, :d + st.cen_x.lo_rows]
    for i in st.layers:
        ay, s1y = _operand(ys[i], st.cen_y[i])
        st.s1y[i] += s1y
        st.sxy[i] += ax[:, :d + 2 * st.cen_x.s].T @ ay[:, :o + st.cen_y[i].lo_rows]
    st.n += x.shape[0]


def rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


def _check(mine, ref):
    # the shifts: the first block's means rounded to fp32 (the device rounds an fp64 sum, torch sums in fp32)
    assert torch.allclose(mine["cx"], ref["cx"].double(), rtol=2.4e-7, atol=0)
    assert torch.allclose(mine["cy"][7], ref["cy"][7].double(), rtol=2.4e-7, atol=0)
    for k in ("sx", "sxx"):
        assert rel(mine[k], ref[k]) < 1e-5, k
    assert rel(mine["sxy"][7], ref["sxy"][7]) < 1e-5 and rel(mine["sy"][7], ref["sy"][7]) < 1e-4


def test_state_recentres_on_the_first_blocks_means():
    x, ys = _data()
    ref = oridge.RidgeStats(3, [7], 16)
    ref.add(x, ys, block=1024)
    ref = ref.state()
    for cap in (ridge.SHIFT_MAX, 3, 0):                 # every channel that qualifies, some, none
        st = ridge.RidgeStats(3, [7], 16, device="cpu", centre_max=cap)
        _emulate(st, x, ys, 1024)
        assert st.cen_x.s == min(cap, st.cen_x.s) and (cap == 0) == (st.cen_x.s == 0)
        mine = st.state()
        _check(mine, ref)
        assert mine["n"] == ref["n"] == 3000
    # the channels chosen are those whose mean exceeds their spread, largest ratio first
    st = ridge.RidgeStats(3, [7], 16, device="cpu", centre_max=3)
    _emulate(st, x, ys, 1024)
    xd = x[:1024].double()
    ratio = xd.mean(0) ** 2 / xd.var(0, unbiased=False)
    assert st.cen_x.idx.tolist() == sorted(ratio.argsort(descending=True)[:3].tolist())


def test_resume_from_a_saved_state():
    x, ys = _data(seed=3)
    ref = oridge.RidgeStats(3, [7], 16)
    ref.add(x, ys, block=1024)
    ref = ref.state()
    first = ridge.RidgeStats(3, [7], 16, device="cpu")
    _emulate(first, x[:1200], {7: ys[7][:1200]}, 1024)
    saved = first.state()
    resumed = ridge.RidgeStats.from_state(saved, device="cpu")
    _emulate(resumed, x[1200:], {7: ys[7][1200:]}, 1024)
    mine = resumed.state()
    assert mine["n"] == 3000 and torch.equal(mine["cx"], saved["cx"])
    _check(mine, ref)


def test_resume_adding_a_subset_of_layers():
    """A resumed state whose new rows add only some layers: state() carries the saved sums of the other layers
    unchanged (their cy, sy, sxy), and the added layer matches the oracle over all rows."""
    x, ys = _data(seed=4)
    ys[9] = (x.float() * 0.5 + 0.25).to(torch.bfloat16)
    ref = oridge.RidgeStats(3, [7], 16)
    ref.add(x, {7: ys[7]}, block=1024)
    ref = ref.state()
    first = ridge.RidgeStats(3, [7, 9], 16, device="cpu")
    _emulate(first, x[:1200], {i: ys[i][:1200] for i in (7, 9)}, 1024)
    saved = first.state()
    resumed = ridge.RidgeStats.from_state(saved, device="cpu")
    resumed.layers = [7]                                # the new rows carry layer 7 only
    _emulate(resumed, x[1200:], {7: ys[7][1200:]}, 1024)
    resumed.layers = [7, 9]
    mine = resumed.state()
    _check(mine, ref)
    for k in ("cy", "sy", "sxy"):
        assert torch.equal(mine[k][9], saved[k][9]), k


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
