"""GPU parity of the closed-form fit at the 8B width of the fit configuration (d 4096, 16 targets,
Student-t(5) rows with 4 outlier channels x 20, Y_l = X T_l + N(0, 0.1), bf16 storage): the device's
sufficient statistics against fp64 products of the same bf16 rows (torch fp64 on the GPU, the checker), and
the maps RidgeFit solves from them against the oracle's fp64 eigendecomposition solve (code/kva/ridge.py:
80-105) of those fp64 statistics, at lambda in {1e-4, 1e-3, 1e-2} x mean(diag C). A second workload adds 8
channels whose mean is 60x their spread (real hidden states carry such channels): the transpose centres them
before the product, and every such channel's sums and the maps stay within the bar; with centring off (raw
sums re-centred in fp64 afterwards) the same channels miss it, so the check has teeth.
Bars: statistics 1e-6 relative Frobenius over each matrix, 1e-5 on the rows, columns and variances of single
channels (fp32 sums over an 8192-row block on MFMA, as the reference's fp32 GEMM); maps 1e-5."""
import pytest
import torch

from oracle import ridge as oridge

pytestmark = pytest.mark.gpu
STAT_TOL, CH_TOL, MAP_TOL = 1e-6, 1e-5, 1e-5
D, TARGETS, ROWS = 4096, 16, 65536
LAMS = (1e-4, 1e-3, 1e-2)


def rel(a, b):
    a, b = a.double(), b.double().to(a.device)
    return float((a - b).norm() / b.norm())


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def workload(dev, targets, rows, shifted=()):
    from rfill import synth
    maps = synth.fit_maps(D, targets, device=dev)
    x, ys = synth.fit_chunk(0, rows, D, maps, device=dev)
    if shifted:
        xf = x.float()
        sd = xf[:, list(shifted)].std(0)
        xf[:, list(shifted)] += 60 * sd                    # mean 60x the spread
        x = xf.to(torch.bfloat16)
        g = torch.Generator(device=dev).manual_seed(77)
        ys = [(x.float() @ t + 0.1 * torch.randn(rows, D, generator=g, device=dev)).to(torch.bfloat16) for t in maps]
    return x, ys


def truth(x, ys, st):
    """fp64 sums of the same bf16 rows about the state's shifts."""
    xd = x.double() - st["cx"].to(x.device)
    out = {"sx": xd.sum(0), "sxx": xd.T @ xd, "sy": {}, "sxy": {}}
    for i, y in enumerate(ys):
        yd = y.double() - st["cy"][i].to(x.device)
        out["sy"][i], out["sxy"][i] = yd.sum(0), xd.T @ yd
        del yd
    return out


def check_maps(st_dev, tr, st, check_targets, dev):
    """RidgeFit on the device statistics vs the oracle's fp64 solve of the fp64 statistics: the worst relative
    error of the weights, and of the bias measured against the size of the terms it is the difference of
    (b = mean_y - mean_x W: with channel means far above their spread b is a small difference of large
    numbers, and any error in W reaches it multiplied by mean_x)."""
    from rfill import ridge
    exact = dict(st, sx=tr["sx"].cpu(), sxx=tr["sxx"].cpu(), sy={i: tr["sy"][i].cpu() for i in check_targets},
                 sxy={i: tr["sxy"][i].cpu() for i in check_targets}, layers=list(check_targets))
    ofit = oridge.RidgeFit(exact)
    fit = ridge.RidgeFit(st_dev, device=dev)
    got = fit.layers(check_targets, LAMS)
    ew = eb = 0.0
    for i in check_targets:
        _, mean_y = ofit.cross(i)
        for lam in LAMS:
            w_ref, b_ref = ofit.layer_f64(i, lam)
            w, b = got[i][lam]
            scale = max(float(b_ref.norm()), float(mean_y.norm()), float((ofit.mean_x @ w_ref.T).norm()))
            ew = max(ew, rel(w.cpu(), w_ref))
            eb = max(eb, float((b.cpu().double() - b_ref).norm()) / scale)
    return ew, eb


def test_transpose_centred_parts_are_exact(dev):
    """rf_transpose_centred against the same split on the CPU: hi, mid and lo bit for bit, hi + mid + lo equal to
    the fp32 x - shift exactly, uncentred columns copied, padding columns zero, column sums and squares."""
    from rfill import ridge
    g = torch.Generator().manual_seed(5)
    rows, cols = 1000, 256
    x = torch.randn(rows, cols, generator=g)
    cen_ch = [3, 17, 64, 200, 255]
    x[:, cen_ch] = x[:, cen_ch] * 0.7 + torch.tensor([50.0, -120.0, 3.3, 1e4, -0.01])
    x = x.to(torch.bfloat16)
    shift = torch.zeros(cols)
    shift[cen_ch] = x[:, cen_ch].float().mean(0)
    lo_row = torch.full((cols,), -1, dtype=torch.int32)
    lo_row[cen_ch] = torch.arange(len(cen_ch), dtype=torch.int32)
    kp = 1024
    dst = torch.full((cols, kp + 64), 7.0, dtype=torch.bfloat16, device=dev)
    lo = torch.full((2 * len(cen_ch), kp + 64), 7.0, dtype=torch.bfloat16, device=dev)
    part = torch.empty(kp // 64, cols, dtype=torch.float32, device=dev)
    sq = torch.empty_like(part)
    ridge.transpose_centred(x.to(dev), dst[:, :kp], lo[:, :kp], shift.to(dev), lo_row.to(dev), part, sq,
                            n_centred=len(cen_ch))
    torch.cuda.synchronize()
    d = x.float() - shift
    hi = d.to(torch.bfloat16)
    r1 = d - hi.float()
    mid = r1.to(torch.bfloat16)
    low = (r1 - mid.float()).to(torch.bfloat16)
    got_hi = dst[:, :rows].cpu().T
    plain = [c for c in range(cols) if c not in cen_ch]
    assert torch.equal(got_hi[:, plain].view(torch.int16), x[:, plain].view(torch.int16))
    assert torch.equal(got_hi[:, cen_ch].view(torch.int16), hi[:, cen_ch].view(torch.int16))
    got_mid, got_lo = lo[:len(cen_ch), :rows].cpu().T, lo[len(cen_ch):, :rows].cpu().T
    assert torch.equal(got_mid.view(torch.int16), mid[:, cen_ch].view(torch.int16))
    assert torch.equal(got_lo.view(torch.int16), low[:, cen_ch].view(torch.int16))
    total = got_hi[:, cen_ch].double() + got_mid.double() + got_lo.double()
    assert torch.equal(total, d[:, cen_ch].double())                       # the three parts sum exactly
    assert bool((dst[:, rows:kp] == 0).all()) and bool((lo[:, rows:kp] == 0).all())
    assert bool((dst[:, kp:] == 7.0).all()) and bool((lo[:, kp:] == 7.0).all())
    s1 = torch.zeros(cols, dtype=torch.float64, device=dev)
    s2 = torch.zeros_like(s1)
    ridge._colsum_fold(part, s1)
    ridge._colsum_fold(sq, s2)
    dd = torch.where(lo_row >= 0, d, x.float()).double()
    assert rel(s1.cpu(), dd.sum(0)) < 1e-6 and rel(s2.cpu(), (dd * dd).sum(0)) < 1e-6


def test_fit_c5_width(dev):
    from rfill import ridge
    x, ys = workload(dev, TARGETS, ROWS)
    stats = ridge.RidgeStats(0, list(range(TARGETS)), D, device=dev)
    stats.add(x, dict(enumerate(ys)))
    st = stats.state(device=dev)
    tr = truth(x, ys, st)
    es = max([rel(st["sxx"], tr["sxx"]), rel(st["sx"], tr["sx"])]
             + [max(rel(st["sxy"][i], tr["sxy"][i]), rel(st["sy"][i], tr["sy"][i])) for i in range(TARGETS)])
    print(f"C5 width: {ROWS} rows, d {D}, {TARGETS} targets, centred channels x {stats.cen_x.s}: "
          f"worst statistics rel err {es:.2e}", flush=True)
    assert es < STAT_TOL
    ew, eb = check_maps(st, tr, stats.state(device="cpu"), (0, 5, 10, 15), dev)
    print(f"C5 width: maps vs the oracle's fp64 solve (lambda {LAMS}): weights {ew:.2e}, bias {eb:.2e}", flush=True)
    assert ew < MAP_TOL and eb < MAP_TOL


@pytest.mark.parametrize("centre", [True, False], ids=["centred", "raw"])
def test_fit_high_mean_channels(dev, centre):
    from rfill import ridge
    shifted = (7, 100, 1000, 2047, 2048, 3000, 4000, 4095)
    x, ys = workload(dev, 2, 32768, shifted)
    stats = ridge.RidgeStats(0, [0, 1], D, device=dev, centre_max=ridge.SHIFT_MAX if centre else 0)
    stats.add(x, dict(enumerate(ys)))
    st = stats.state(device=dev)
    tr = truth(x, ys, st)
    idx = list(shifted)
    per_ch = max([rel(st["sxx"][idx], tr["sxx"][idx])] + [rel(st["sxy"][i][idx], tr["sxy"][i][idx]) for i in (0, 1)]
                 + [rel(st["sxy"][i][:, idx], tr["sxy"][i][:, idx]) for i in (0, 1)])
    diag = float(((st["sxx"].diagonal()[idx] - tr["sxx"].diagonal()[idx]).abs() / tr["sxx"].diagonal()[idx]).max())
    print(f"high-mean channels ({'centred' if centre else 'raw sums'}): centred x channels {stats.cen_x.s}, "
          f"their rows / columns rel err {per_ch:.2e}, worst variance rel err {diag:.2e}", flush=True)
    if not centre:
        assert per_ch > 10 * CH_TOL or diag > 10 * CH_TOL         # raw sums miss the bar on these channels
        return
    assert set(idx) <= set(stats.cen_x.idx.tolist())
    assert per_ch < CH_TOL and diag < CH_TOL
    ew, eb = check_maps(st, tr, stats.state(device="cpu"), (0, 1), dev)
    print(f"high-mean channels: maps vs the oracle's fp64 solve: weights {ew:.2e}, bias {eb:.2e}", flush=True)
    assert ew < MAP_TOL and eb < MAP_TOL
