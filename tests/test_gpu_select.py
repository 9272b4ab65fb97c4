"""The qattn selector on the device: rf_window_mass against a float64 computation from the same queries and
keys (dense causal softmax, summed over window rows and query heads) at an 8B-class shape and at a small
head_dim-64 case with the window ending before the cache's end; rfill.select.window_mass (queries by
rf_norm_q, mass by rf_window_mass) against the oracle's window_mass on the same model and cache, and
the rows it selects; the refusals."""
import pytest
import torch

from fill_cases import case, inputs, rel_err
from oracle import model as OM
from oracle import select as OS

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def mass64(q, k, pos0, scale):
    """float64 reference: q [w, hq d], k [hkv, n, d] -> [n]."""
    w = q.shape[0]
    hkv, n, d = k.shape
    hq = q.shape[1] // d
    qh = q.double().view(w, hq, d).transpose(0, 1)                   # [hq, w, d]
    kk = k.double().repeat_interleave(hq // hkv, 0)                    # [hq, n, d]
    s = torch.matmul(qh, kk.transpose(1, 2)) * scale
    s.masked_fill_(torch.arange(n)[None, None, :] > (pos0 + torch.arange(w))[None, :, None], float("-inf"))
    return torch.softmax(s, -1).sum((0, 1))


@pytest.mark.parametrize("n,w,end,hq,hkv,d", [(4096, 64, 4096, 32, 8, 128), (1000, 16, 700, 8, 4, 64),
                                               (3000, 64, 2900, 16, 2, 256)])
def test_window_mass_kernel(dev, n, w, end, hq, hkv, d):
    from rfill import ops
    g = torch.Generator().manual_seed(n)
    q = (0.5 * torch.randn(w, hq * d, generator=g)).to(torch.bfloat16)
    kb = torch.zeros(hkv, n + 64, d, dtype=torch.bfloat16)
    kb[:, :n] = (0.5 * torch.randn(hkv, n, d, generator=g)).to(torch.bfloat16)
    mass = torch.zeros(n, dtype=torch.float64, device=dev)
    ops.window_mass(q.to(dev), end - w, kb.to(dev), hq, d ** -0.5, mass)
    torch.cuda.synchronize()
    want = mass64(q, kb[:, :n], end - w, d ** -0.5)
    got = mass.cpu()
    err = float((got - want).norm() / want.norm())
    print(f"window mass {n} keys, {w} rows, {hq}/{hkv} heads, d {d}: rel err {err:.2e}, sum {got.sum():.3f}")
    assert err < 1e-5
    assert abs(float(got.sum()) - w * hq) < 1e-3 * w * hq
    assert bool((got[end:] == 0).all())


def test_select_matches_oracle(dev):
    """Lower layers 1 and 3 of a small Llama filled from the same inputs on both sides; the last 64 rows
    as the window."""
    from rfill.model import FillModel
    from rfill import select as RS
    cfg, t = case("llama_c1", layers=4)
    n, w, layers = 2048, 64, [1, 3]
    pos = torch.arange(n)
    xs = {L: inputs(n, cfg["hidden_size"], seed=60 + L) for L in layers}
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    m = FillModel(cfg, t, dev, layers=layers)
    c = m.new_cache()
    for L in layers:
        om.fill(L, xs[L], pos, oc)
        m.fill(L, xs[L].to(dev), pos.to(dev), c)
    want = OS.window_mass(om, {L: xs[L][n - w:] for L in layers}, oc, layers)
    got = RS.window_mass(m, {L: xs[L][n - w:].to(dev) for L in layers}, c, layers)
    err = rel_err(got, want)
    b = round(0.05 * n)
    rg, rw = set(RS.top_rows(got, n - 256, b)), set(OS.top_rows(want, n - 256, b))
    jac = len(rg & rw) / len(rg | rw)
    print(f"window mass vs the oracle: rel err {err:.2e}; top {b} rows of [0, {n - 256}) Jaccard {jac:.3f}")
    assert err < 1e-2 and jac > 0.9
    assert abs(float(got.sum()) - len(layers) * w * m.n_heads) < 1e-3 * len(layers) * w * m.n_heads


def test_window_mass_refuses(dev):
    from rfill import ops
    q = torch.zeros(10, 4 * 64, dtype=torch.bfloat16, device=dev)
    kb = torch.zeros(2, 200, 64, dtype=torch.bfloat16, device=dev)
    mass = torch.zeros(200, dtype=torch.float64, device=dev)
    with pytest.raises(ValueError):          # 2 heads per K / V head x 10 rows is not a multiple of 32
        ops.window_mass(q, 100, kb, 4, 0.125, mass)
    with pytest.raises(ValueError):
        ops.window_mass(q[:8], 195, kb, 4, 0.125, mass)      # past the cache


def test_select_on_a_hybrid(dev):
    """The qattn mass at the attention layer of a Qwen3.5 hybrid (gated queries, zero-centred q_norm,
    partial RoPE, head_dim 256): layer 3 filled from the same inputs on both sides."""
    from fill_cases import hybrid_config, hybrid_tensors
    from rfill.model import FillModel
    from rfill import select as RS
    cfg = hybrid_config(["gdn", "gdn", "gdn", "attn"], hidden=512, hkv=2, d=256)
    t = hybrid_tensors(cfg, seed=9)
    n, w, layers = 1500, 64, [3]
    pos = torch.arange(n)
    x = inputs(n, cfg["hidden_size"], seed=63)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    om.fill(3, x, pos, oc)
    m = FillModel(cfg, t, dev)
    c = m.new_cache()
    m.fill(3, x.to(dev), pos.to(dev), c)
    want = OS.window_mass(om, {3: x[n - w:]}, oc, layers)
    got = RS.window_mass(m, {3: x[n - w:].to(dev)}, c, layers)
    err = rel_err(got, want)
    print(f"hybrid window mass vs the oracle: rel err {err:.2e}")
    assert err < 1e-2
    assert abs(float(got.sum()) - w * m.n_heads) < 1e-3 * w * m.n_heads
