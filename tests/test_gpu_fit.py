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


@pytest.mark.parametrize("M,N,K,fold_rows", [(4104, 4352, 12288, 8192), (4352, 4096, 16384, 4096)])
def test_gram_run_split_schedule_is_bit_identical(dev, M, N, K, fold_rows):
    """Tile counts just past one round of the GPU's 256 CUs (a centred operand's extra rows / columns: 289
    and 272 tiles): with a workspace the tiles past the first 256 run as single runs whose fp32 sums a second
    kernel adds into C in run order. The same bits as every tile whole (no workspace, or one a byte short),
    nothing written past the workspace (a guard region after it), and fp64 products to 1e-6; the first
    shape's last run is shorter than fold_rows (12288 = 8192 + 4096)."""
    from rfill import _lib, ridge
    from rfill.ops import _ptr, _stream
    need = ridge.gram_workspace_bytes(M, N, K, fold_rows)
    assert need > 0
    g = torch.Generator(device=dev).manual_seed(3)
    a = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    b = (torch.randn(N, K, generator=g, device=dev) * 2).to(torch.bfloat16)
    c0 = torch.randn(M, N, generator=g, device=dev, dtype=torch.float64)
    whole = c0.clone()
    _lib.call("rf_gram_accumulate", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, fold_rows, _ptr(whole),
              whole.stride(0), None, 0, _stream(a))
    guard = 1 << 20
    buf = torch.full((need + guard,), 0xFF, dtype=torch.uint8, device=dev)     # stale contents must not matter
    split = c0.clone()
    _lib.call("rf_gram_accumulate", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, fold_rows, _ptr(split),
              split.stride(0), _ptr(buf), need, _stream(a))
    short = c0.clone()                                                  # one byte short: every tile whole
    _lib.call("rf_gram_accumulate", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, fold_rows, _ptr(short),
              short.stride(0), _ptr(buf), need - 1, _stream(a))
    torch.cuda.synchronize()
    assert torch.equal(split, whole) and torch.equal(short, whole)
    assert bool((buf[need:] == 0xFF).all()), "the run-split schedule wrote past its workspace"
    err = rel(split - c0, a.double() @ b.double().T)
    print(f"gram {M} x {N} x {K} (fold {fold_rows}) run-split rel err {err:.2e}")
    assert err < 1e-6


@pytest.mark.parametrize("M,N,K,fold_rows", [(4104, 4352, 16384, 8192), (1024, 1024, 12288, 8192),
                                              (768, 1024, 2048, 0)])
def test_gram_upper_is_the_full_product_on_its_tiles(dev, M, N, K, fold_rows):
    """The symmetric X^T X on C's block-upper tiles (a centred X's 4104 rows against its 4352-row operand: 153
    of 289 tiles, each split into its two runs; a short last run; one run, whole tiles): those tiles
    bit-identical to rf_gram_accumulate of the same operands, the block-lower tiles untouched, the same bits
    with no workspace, nothing written past the workspace, and after mirror_block_upper the full product
    (fp64 products to 1e-6; the full launch's own lower tiles differ from the mirrored upper ones by fp32
    summation order only, about 1e-13 of C here)."""
    from rfill import _lib, ridge
    from rfill.ops import _ptr, _stream
    g = torch.Generator(device=dev).manual_seed(5)
    a = torch.randn(N, K, generator=g, device=dev).to(torch.bfloat16)
    a[M:] = 0                                                           # rows past M: a centred operand's padding
    c0 = torch.randn(M, N, generator=g, device=dev, dtype=torch.float64)
    c0[:, :M] += c0[:, :M].T.clone()                                    # a symmetric running sum, as RidgeStats'
    full = c0.clone()
    ridge.gram_accumulate(a[:M], a, full, fold_rows)
    need = ridge.gram_upper_workspace_bytes(M, N, K, fold_rows)
    assert (need > 0) == (fold_rows > 0)
    guard = 1 << 20
    buf = torch.full((need + guard,), 0xFF, dtype=torch.uint8, device=dev)
    up = c0.clone()
    _lib.call("rf_gram_accumulate_upper", _ptr(a), a.stride(0), M, N, K, fold_rows, _ptr(up), up.stride(0),
              _ptr(buf), need, _stream(a))
    whole = c0.clone()
    ridge.gram_accumulate_upper(a, M, whole, fold_rows, torch.empty(0, dtype=torch.uint8, device=dev))
    torch.cuda.synchronize()
    assert bool((buf[need:] == 0xFF).all()), "the upper schedule wrote past its workspace"
    assert torch.equal(whole, up)
    ti = torch.arange(M, device=dev)[:, None] // 256
    tj = torch.arange(N, device=dev)[None, :] // 256
    upper = tj >= ti
    assert torch.equal(up[upper], full[upper])
    assert torch.equal(up[~upper], c0[~upper])
    ridge.mirror_block_upper(up)
    sym = full[:, :M] - c0[:, :M]
    asym = float((sym - sym.T).abs().max())
    print(f"gram upper {M} x {N} x {K} (fold {fold_rows}): full product symmetric to {asym:.1e}")
    d = a[:M].double()
    want = d @ a.double().T
    assert torch.equal(up[:, M:], c0[:, M:])                           # products with the zero rows
    low = ~upper[:, :M]
    assert torch.equal(up[:, :M][low], (up[:, :M].T)[low])
    err = rel(up[:, :M][low] - c0[:, :M][low], want[:, :M][low])
    assert err < 1e-6, err


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


def _centred(st, i):
    """Shift-free statistics of a state: the means of x and y_i, C = sxx - sx sx^T / n, Cxy = sxy - sx sy^T / n."""
    n = float(st["n"])
    sx, sy = st["sx"].double().cpu(), st["sy"][i].double().cpu()
    return dict(mx=st["cx"].double().cpu() + sx / n, my=st["cy"][i].double().cpu() + sy / n,
                c=st["sxx"].double().cpu() - torch.outer(sx, sx) / n,
                cxy=st["sxy"][i].double().cpu() - torch.outer(sx, sy) / n)


def test_resumed_statistics_continue_the_device_sums(dev):
    """RidgeStats.from_state on the device (the reference's resumable sufficient statistics,
    code/scripts/fit_sweep.py:20-25, :271-284): a state saved after the first 7000 rows, moved to the host
    and back as a saved file would be, then continued with the remaining rows, keeps the saved shifts and
    gives one pass's means, centred scatter and centred cross products (1e-6); a resume that adds layer 5
    only carries layer 6's saved sums unchanged; maps fitted from the resumed state agree with one pass's
    (1e-5)."""
    from rfill import ridge
    n, d = 20000, 512
    x = _student(n, d, 7)
    g = torch.Generator().manual_seed(8)
    ys = {}
    for i in (5, 6):
        t = torch.eye(d) + 0.05 * torch.randn(d, d, generator=g) / d ** 0.5
        ys[i] = (x.float() @ t + 0.1 * torch.randn(n, d, generator=g)).to(torch.bfloat16)
    xd, yd = x.to(dev), {i: y.to(dev) for i, y in ys.items()}
    one = ridge.RidgeStats(4, [5, 6], d, device=dev)
    one.add(xd, yd, block=8192)
    want = one.state()
    first = ridge.RidgeStats(4, [5, 6], d, device=dev)
    first.add(xd[:7000], {i: y[:7000] for i, y in yd.items()}, block=8192)
    saved = first.state(device="cpu")
    resumed = ridge.RidgeStats.from_state(saved, device=dev)
    resumed.add(xd[7000:], {i: y[7000:] for i, y in yd.items()}, block=8192)
    got = resumed.state()
    assert got["n"] == n and torch.equal(got["cx"].cpu(), saved["cx"].cpu())
    for i in (5, 6):
        assert torch.equal(got["cy"][i].cpu(), saved["cy"][i].cpu())
    # the shifts differ (the first 8192-row block's means against the first 7000 rows'), so compare the
    # statistics every shift gives alike: means, centred scatter and centred cross products
    for (k, a), (_, b) in zip(_centred(got, 5).items(), _centred(want, 5).items()):
        assert rel(a, b) < 1e-6, (k, rel(a, b))
    for (k, a), (_, b) in zip(_centred(got, 6).items(), _centred(want, 6).items()):
        assert rel(a, b) < 1e-6, (k, rel(a, b))
    part = ridge.RidgeStats.from_state(saved, device=dev)
    part.begin(xd[7000:], block=8192)
    part.add_layer(5, yd[5][7000:])
    ps = part.state()
    assert rel(_centred(ps, 5)["cxy"], _centred(want, 5)["cxy"]) < 1e-6
    for k in ("cy", "sy", "sxy"):
        assert torch.equal(ps[k][6].cpu(), saved[k][6].cpu()), k
    fa, fb = ridge.RidgeFit(got, device=dev), ridge.RidgeFit(want, device=dev)
    for lam in (1e-3, 1e-2):
        wa, ba = fa.layer(6, (lam,))[lam]
        wb, bb = fb.layer(6, (lam,))[lam]
        assert rel(wa, wb) < 1e-5 and rel(ba, bb) < 1e-5
