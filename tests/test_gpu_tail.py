"""GPU parity of the exact tail (FillModel.layer: the tail rows' K / V appended after the filled rows,
causal attention over the whole cache, o_proj, MLP; code/kva/model.py:247-257), of the final norm +
lm_head logits (code/kva/model.py:110-111) and of finish() composed from them (the late layers of
code/kva/kva.py:319-460) against the CPU oracle on identical seeded inputs.

Bars: outputs, caches and logits within relative Frobenius error 1e-2 (bf16 path); cache lengths and
slots exact."""
import pytest
import torch

from fill_cases import case, inputs, rel_err
from oracle import kva as OK
from oracle import model as OM

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.mark.parametrize("name", ["llama_c1", "llama3_scaled", "qwen3_knorm"])
def test_layer_matches_oracle(dev, name):
    """P filled rows, then T tail rows through the exact layer: the tail's output, its K / V slots
    [P, P + T) and the untouched prefix slots against the oracle."""
    from rfill.model import FillModel
    cfg, t = case(name)
    P, T, H = 1000, 300, cfg["hidden_size"]
    x = inputs(P, H, seed=31)
    h = inputs(T, H, seed=32)
    pos = torch.arange(P + T)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    om.fill(0, x, pos[:P], oc)
    want = om.layer(0, h, pos[P:], oc)
    m = FillModel(cfg, t, dev)
    c = m.new_cache()
    m.fill(0, x.to(dev), pos[:P].to(dev), c)
    got, ssq = m.layer(0, h.to(dev), pos[P:].to(dev), c)
    torch.cuda.synchronize()
    assert c[0]["n"] == P + T and c[0]["k"].shape[1] == P + T
    err = rel_err(got, want)
    ed = rel_err(got.cpu().float() - h.float(), want.float() - h.float())       # the layer's own update
    ek = rel_err(c[0]["k"][:, P:], oc[0]["k"][:, P:])
    ev = rel_err(c[0]["v"][:, P:], oc[0]["v"][:, P:])
    ep = rel_err(c[0]["k"][:, :P], oc[0]["k"][:, :P])
    # the returned statistics are the output's own row sums of squares (the next norm's input)
    es = rel_err(ssq.sum(1), got.float().pow(2).sum(1))
    print(f"{name}: tail out {err:.2e}, update {ed:.2e}, tail K {ek:.2e} V {ev:.2e}, prefix K {ep:.2e}, ssq {es:.1e}")
    # The update (output - input) is about 0.2 of the input's norm here, so the output's own bf16 rounding
    # moves it by 8e-3 (measured on the CPU: the fp32 oracle's output rounded to bf16), and the bf16
    # oracle sits 1.3e-2 from the fp32 one; its bar is therefore 2e-2, the output's stays 1e-2.
    assert err < TOL and ed < 2 * TOL and ek < TOL and ev < TOL and ep < TOL and es < 1e-5


def test_logits_match_oracle(dev):
    from rfill.model import FillModel
    cfg, t = case("qwen3_knorm")
    h = inputs(77, cfg["hidden_size"], seed=33)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    want = om.logits(h)
    got = FillModel(cfg, t, dev).logits(h.to(dev))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and got.shape == want.shape
    err = rel_err(got, want)
    print(f"logits rel err {err:.2e}")
    assert err < TOL
    assert (got.argmax(-1).cpu() == want.argmax(-1)).float().mean() > 0.9


@pytest.mark.parametrize("exact", [False, True])
def test_finish_matches_oracle(dev, exact):
    """The whole late stack of one ridgefill arm: fill of every late layer (with 18 exact rows run
    through their layers, or none), the 256-row exact tail through every late layer, tail logits."""
    from rfill.kva import Arm, Projector, finish
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=8)
    N, tail, split, keep = 2048, 256, 5, 100
    P, H = N - tail, cfg["hidden_size"]
    h = inputs(N, H, seed=14)
    g = torch.Generator().manual_seed(15)
    W = {i: (torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16)
         for i in range(split, 8)}
    B = {i: (1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for i in range(split, 8)}
    rows = torch.randperm(P, generator=g)[:18].sort().values if exact else None
    m = FillModel(cfg, t, dev)
    arm = Arm("ridgefill", split=split, tail=tail, fill="proj", projector=Projector(split, W, B))
    logits, cache, P_got = finish(m, torch.zeros(N, dtype=torch.long), h.to(dev), None, arm, keep, exact_rows=rows)
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oarm = OK.Arm("ridgefill", split=split, tail=tail, fill="proj", projector=OK.Projector(split, W, B))
    want, oc, P_want = OK.finish(om, torch.zeros(N, dtype=torch.long), h, om.new_cache(), oarm, keep,
                                 exact_rows=rows)
    assert P_got == P_want == P and logits.shape == want.shape
    el = rel_err(logits, want)
    worst = 0.0
    for i in range(split, 8):
        assert cache[i]["n"] == N
        for part in ("k", "v"):
            worst = max(worst, rel_err(cache[i][part], oc[i][part]))
    agree = float((logits.argmax(-1).cpu() == want.argmax(-1)).float().mean())
    print(f"finish (exact rows: {exact}): logits rel err {el:.2e}, argmax agreement {agree:.3f}, worst K/V {worst:.2e}")
    assert el < TOL and worst < TOL and agree > 0.9


def test_finish_refuses(dev):
    from rfill.kva import Arm, finish
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=2)
    m = FillModel(cfg, t, dev)
    h = inputs(300, cfg["hidden_size"], seed=3).to(dev)
    ids = torch.zeros(300, dtype=torch.long)
    with pytest.raises(ValueError):
        finish(m, ids, h, None, Arm("x", split=1, tail=50, fill="identity"), keep=51)      # keep > tail
    with pytest.raises(ValueError):
        finish(m, ids, h, None, Arm("x", split=1, tail=50, fill="oracle"), keep=10)


def test_finish_exact_arm_is_the_exact_layer_stack(dev):
    """The exact arm (P = 0): every row runs the exact late layers; the same as layer() by hand."""
    from rfill.kva import Arm, finish
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=3)
    m = FillModel(cfg, t, dev)
    h = inputs(200, cfg["hidden_size"], seed=4).to(dev)
    logits, cache, P = finish(m, torch.zeros(200, dtype=torch.long), h, None, Arm("exact", split=1, fill="exact"), keep=20)
    c2 = m.new_cache()
    x = h
    pos = torch.arange(200, device=dev)
    for i in (1, 2):
        x, _ = m.layer(i, x, pos, c2)
    torch.cuda.synchronize()
    assert P == 0 and cache[2]["n"] == 200
    assert torch.equal(logits, m.logits(x[-20:]))
