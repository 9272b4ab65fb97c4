"""GPU parity of the closed-form fit: rf_transpose (bit-exact, column sums), rf_gram_accumulate (fp32
over the block into fp64), RidgeStats on the device against the oracle's RidgeStats, and RidgeFit's
fp64 solve against the oracle's fp64 eigendecomposition solve. Bar for fitted maps: relative Frobenius
error <= 1e-5 against the fp64 reference solve."""
import pytest
import torch

from oracle import ridge as oridge

pytestmark = pytest.mark.gpu
MAP_TOL = 1e-5


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch.device("cuda")


def test_transpose_is_bit_exact_with_column_sums(dev):
    from rfill import ridge
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1000, 512, generator=g).to(torch.bfloat16).to(dev)
    dst = torch.full((512, 1088), 5.0, dtype=torch.bfloat16, device=dev)
    part = torch.empty(1024 // 64, 512, dtype=torch.float32, device=dev)
    ridge._transpose(x, dst[:, :1024], part)
    torch.cuda.synchronize()
    assert torch.equal(dst[:, :1000], x.T)
    assert bool((dst[:, 1000:1024] == 0).all()) and bool((dst[:, 1024:] == 5.0).all())
    sums = torch.zeros(512, dtype=torch.float64, device=dev)
    ridge._colsum_fold(part, sums)
    assert rel(sums, x.double().sum(0)) < 1e-6


@pytest.mark.parametrize("fold_rows", [0, 128, 512])
def test_gram_accumulate_matches_fp64_products(dev, fold_rows):
    """fp32 runs of at most fold_rows added into fp64 in run order, against fp64 products; fold_rows 0 sums
    the whole K in fp32. The same bits run to run."""
    from rfill import ridge
    g = torch.Generator().manual_seed(1)
    a = torch.randn(384, 1024, generator=g).to(torch.bfloat16)
    b = (torch.randn(768, 1024, generator=g) * 3).to(torch.bfloat16)
    c0 = torch.randn(384, 768, generator=g, dtype=torch.float64)
    c = c0.to(dev)
    ridge.gram_accumulate(a.to(dev), b.to(dev), c, fold_rows)
    want = c0 + a.double() @ b.double().T
    err = rel(c, want)
    print(f"gram (fold_rows {fold_rows}) rel err {err:.2e}")
    assert err < 1e-6
    again = c0.to(dev)
    ridge.gram_accumulate(a.to(dev), b.to(dev), again, fold_rows)
    assert torch.equal(again, c)


def test_gram_accumulate_refuses_bad_fold(dev):
    from rfill import ridge
    a = torch.zeros(256, 128, dtype=torch.bfloat16, device=dev)
    c = torch.zeros(256, 256, dtype=torch.float64, device=dev)
    with pytest.raises(ValueError, match="fold_rows"):
        ridge.gram_accumulate(a, a, c, 96)


def _student(n, d, seed):
    from rfill import synth
    g = torch.Generator().manual_seed(seed)
    x = synth.student_t((n, d), 5, g, "cpu")
    x[:, :4] *= 20
    return x.to(torch.bfloat16)


def test_ridge_stats_and_fit_match_the_oracle(dev):
    """Config-5-shaped data at a reduced size (d 512, 2 targets, 20000 rows, ragged last block): the
    device statistics against the oracle's (fp32 block GEMMs into fp64), and the maps fitted from each
    against the oracle's fp64 solve."""
    from rfill import ridge
    n, d = 20000, 512
    x = _student(n, d, 2)
    g = torch.Generator().manual_seed(3)
    ys = {}
    for i in (5, 6):
        t = torch.eye(d) + 0.05 * torch.randn(d, d, generator=g) / d ** 0.5
        ys[i] = (x.float() @ t + 0.1 * torch.randn(n, d, generator=g)).to(torch.bfloat16)
    mine = ridge.RidgeStats(4, [5, 6], d, device=dev)
    mine.add(x.to(dev), {i: y.to(dev) for i, y in ys.items()}, block=8192)
    ms = mine.state()
    ref = oridge.RidgeStats(4, [5, 6], d)
    ref.add(x, ys, block=8192)
    rs = ref.state()
    for k in ("sx", "sxx"):
        print(k, rel(ms[k], rs[k]))
        assert rel(ms[k], rs[k]) < 1e-5, k
    for i in (5, 6):
        assert rel(ms["sxy"][i], rs["sxy"][i]) < 1e-5
    ofit = oridge.RidgeFit(rs)
    same = ridge.RidgeFit(rs, device=dev)           # the solve alone, on the oracle's statistics
    full = ridge.RidgeFit(ms, device=dev)           # device statistics + device solve
    for lam in (1e-4, 1e-3, 1e-2):
        w_ref, b_ref = ofit.layer_f64(6, lam)
        w1, b1 = same.layer(6, (lam,))[lam]
        w2, b2 = full.layer(6, (lam,))[lam]
        e1, e2 = rel(w1, w_ref), rel(w2, w_ref)
        print(f"lam {lam:g}: solve-only rel err {e1:.2e}, stats+solve rel err {e2:.2e}")
        assert e1 < MAP_TOL and rel(b1, b_ref) < MAP_TOL
        assert e2 < MAP_TOL
