"""GPU parity of the fit driver (code/scripts/fit_sweep.py:62-166, :236-318): rf_read_cosine against an
fp64 cosine, FillModel.forward_exact against the oracle's exact forward, the capture sums against the
oracle's Capture fed the same layer inputs (state tolerance 1e-5 relative Frobenius, as the fit's
statistics), and the held-out read-cosine scores against the oracle's scores on the same maps (2e-4
absolute: the two forwards differ by bf16 roundings; measured 3e-5), with the same chosen lambda."""
import pytest
import torch

from fill_cases import case, rel_err
from oracle import fit as OF
from oracle import model as OM
from oracle import ridge as oridge

pytestmark = pytest.mark.gpu
STAT_TOL = 1e-5
SCORE_TOL = 2e-4


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _cos64(a, b, hkv, d, gain):
    """Sum over rows and heads of the K and V cosines, fp64 on the CPU."""
    a, b = a.double().view(a.shape[0], 2, hkv, d), b.double().view(b.shape[0], 2, hkv, d)
    out = []
    for kind in (0, 1):
        x, y = a[:, kind], b[:, kind]
        if kind == 0 and gain is not None:
            x, y = x * gain, y * gain
        num = (x * y).sum(-1)
        den = x.norm(dim=-1).clamp_min(1e-8) * y.norm(dim=-1).clamp_min(1e-8)
        out.append(float((num / den).sum()))
    return out


@pytest.mark.parametrize("rows,hkv,d,gk", [(1000, 2, 64, None), (37, 8, 128, 0), (500, 1, 256, 1), (16, 4, 128, None)])
def test_read_cosine_matches_fp64(dev, rows, hkv, d, gk):
    from rfill import ops
    g = torch.Generator().manual_seed(rows + d)
    t = torch.randn(rows, 2 * hkv * d + 64, generator=g).to(torch.bfloat16)
    p = (t.float() + 0.3 * torch.randn(t.shape, generator=g)).to(torch.bfloat16)
    p[3 % rows, :d] = 0                           # a zero K head: cosine 0 (the norm's eps clamp)
    gain = None if gk is None else (1 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16)
    out = torch.zeros(2, dtype=torch.float64, device=dev)
    w = 1.0 / (rows * hkv)
    for _ in range(2):                            # accumulates
        ops.read_cosine(p.to(dev), t.to(dev), hkv, hkv, d, None if gain is None else gain.to(dev), gk or 0, w, out)
    torch.cuda.synchronize()
    gw = None if gain is None else gain.double() + (1.0 if gk == 1 else 0.0)
    want = _cos64(p[:, :2 * hkv * d], t[:, :2 * hkv * d], hkv, d, gw)
    got = out.cpu().tolist()
    print(f"rows {rows} hkv {hkv} d {d}: got {got}, want {[2 * w * x for x in want]}")
    for a, b in zip(got, want):
        assert abs(a - 2 * w * b) < 1e-6


@pytest.mark.parametrize("rows,na,nb,d", [(300, 3, 0, 8), (77, 2, 5, 16), (129, 1, 0, 64), (40, 4, 4, 32)])
def test_read_cosine_groups_match_fp64(dev, rows, na, nb, d):
    """Unequal groups and narrow vectors (a GDN layer's v heads alone, its [b | a] row of 2 nv values): group
    a's sum into out[0] with its gain, group b's into out[1]; with nb = 0 out[1] stays untouched."""
    from rfill import ops
    g = torch.Generator().manual_seed(rows + na)
    t = torch.randn(rows, (na + nb) * d + 8, generator=g).to(torch.bfloat16)
    p = (t.float() + 0.5 * torch.randn(t.shape, generator=g)).to(torch.bfloat16)
    gain = (1 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16)
    out = torch.full((2,), 7.0, dtype=torch.float64, device=dev)
    ops.read_cosine(p.to(dev), t.to(dev), na, nb, d, gain.to(dev), 0, 0.5, out)
    torch.cuda.synchronize()
    a, b = p[:, :(na + nb) * d].double().view(rows, na + nb, d), t[:, :(na + nb) * d].double().view(rows, na + nb, d)
    a[:, :na] *= gain.double()
    b[:, :na] *= gain.double()
    cos = (a * b).sum(-1) / (a.norm(dim=-1).clamp_min(1e-8) * b.norm(dim=-1).clamp_min(1e-8))
    want = [7.0 + 0.5 * float(cos[:, :na].sum()), 7.0 + (0.5 * float(cos[:, na:].sum()) if nb else 0.0)]
    got = out.cpu().tolist()
    assert abs(got[0] - want[0]) < 1e-5 * max(1.0, abs(want[0])) and abs(got[1] - want[1]) < 1e-5 * max(1.0, abs(want[1]))


def test_read_cosine_refuses(dev):
    from rfill import _lib
    x = torch.zeros(16, 2 * 96, dtype=torch.bfloat16, device=dev)
    out = torch.zeros(2, dtype=torch.float64, device=dev)
    ws = torch.empty(64, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="a power of two"):
        _lib.call("rf_read_cosine", x.data_ptr(), 192, x.data_ptr(), 192, 16, 1, 1, 96, None, 0, 1.0, out.data_ptr(),
                  ws.data_ptr(), 64, None)
    x = torch.zeros(40, 256, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("rf_read_cosine", x.data_ptr(), 256, x.data_ptr(), 256, 40, 1, 1, 128, None, 0, 1.0, out.data_ptr(),
                  ws.data_ptr(), 16, None)


def _docs(n_list, seed, vocab=64):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (n,), generator=g) for n in n_list]


@pytest.mark.parametrize("name", ["llama_c1", "qwen3_knorm"])
def test_forward_exact_matches_oracle(dev, name):
    from rfill.model import FillModel
    cfg, t = case(name, layers=4)
    ids = _docs([300], 11)[0]
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    want, mine = {}, {}
    lw, _ = om.forward_exact(ids, hook=lambda i, h: want.__setitem__(i, h), keep=[0, 150, 299])
    m = FillModel(cfg, t, dev)
    lg, cache = m.forward_exact(ids, hook=lambda i, h: mine.__setitem__(i, h.clone()), keep=[0, 150, 299])
    torch.cuda.synchronize()
    assert all(c["n"] == 300 for c in cache)
    assert torch.equal(mine[0].cpu(), want[0])                     # the embedding gather is exact
    errs = {i: rel_err(mine[i], want[i]) for i in (1, 2, 3, "final")}
    el = rel_err(lg, lw)
    print(f"{name}: layer inputs {errs}, logits {el:.2e}")
    assert all(e < 2e-2 for e in errs.values()) and el < 2e-2
    # stop: the hook of layer `stop` is the last, with the same rows
    seen = []
    m.forward_exact(ids, hook=lambda i, h: seen.append((i, h.clone())), stop=2)
    assert [i for i, _ in seen] == [0, 1, 2] and torch.equal(seen[2][1], mine[2])


@pytest.mark.parametrize("name,splits,block", [("llama_c1", [1, 2], 512), ("qwen3_knorm", [2], 8192)])
def test_capture_sums_match_the_oracle(dev, name, splits, block):
    """Ragged documents (one longer than the block: the block grows), sums against the oracle's Capture
    fed the device's own layer inputs (the forward is checked above)."""
    from rfill import fit
    from rfill.model import FillModel
    cfg, t = case(name, layers=4)
    m = FillModel(cfg, t, dev)
    docs = _docs([300, 77, 700, 129], 12)
    cap = fit.Capture(m, splits, block=block)
    ref = oridge.Capture(splits, 4, cfg["hidden_size"])
    for ids in docs:
        cap.add_document(ids)
        got = {}
        m.forward_exact(ids, hook=lambda i, h: got.__setitem__(i, h.float().cpu()) if i != "final" and i >= min(splits)
                        else None)
        ref.add_document(got)
    for S in splits:
        a, b = cap.state(S), ref.state(S)
        assert a["n"] == b["n"] == 1206 and a["layers"] == b["layers"] == list(range(S, 4))
        errs = dict(cx=rel_err(a["cx"], b["cx"]), sx=rel_err(a["sx"], b["sx"]), sxx=rel_err(a["sxx"], b["sxx"]))
        for i in a["layers"]:
            errs[f"cy{i}"] = rel_err(a["cy"][i], b["cy"][i])
            errs[f"sy{i}"] = rel_err(a["sy"][i], b["sy"][i])
            errs[f"sxy{i}"] = rel_err(a["sxy"][i], b["sxy"][i])
        print(f"{name} S={S}: " + ", ".join(f"{k} {v:.1e}" for k, v in errs.items()))
        assert all(v < STAT_TOL for v in errs.values()), errs


def test_selection_matches_the_oracle(dev):
    """Device fit + held-out scores against the oracle's scores of the same maps over its own bf16
    forward; the identity scores 1 at the split layer; fit_sweep returns the chosen lambda's maps."""
    from rfill import fit
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=4)
    m = FillModel(cfg, t, dev)
    docs, held = _docs([400, 260, 333, 150], 13), _docs([200, 333], 14)
    lams = (1e-4, 1e-2, 1.0)
    S = 2
    cap = fit.Capture(m, [S])
    for ids in docs:
        cap.add_document(ids)
    maps = fit.fit_maps(cap.state(S, device=dev), lams, device=dev)
    mine = fit.read_scores(m, held, S, maps)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    cpu_maps = {lam: {i: (w.cpu(), b.cpu()) for i, (w, b) in per.items()} for lam, per in maps.items()}
    want = OF.read_scores(om, held, S, cpu_maps)
    worst = max(abs(mine[c][i] - want[c][i]) for c in want for i in want[c])
    print("scores (device / oracle):", {c: [(round(mine[c][i], 5), round(want[c][i], 5)) for i in mine[c]]
                                       for c in mine}, f"worst {worst:.1e}")
    assert worst < SCORE_TOL
    assert abs(mine["identity"][S] - 1.0) < 1e-6
    mean = {c: sum(v.values()) / len(v) for c, v in want.items()}
    top = sorted((mean[lam] for lam in lams), reverse=True)
    if top[0] - top[1] > 2 * SCORE_TOL:
        assert fit.best_lambda(mine, lams) == OF.best_lambda(want, lams)
    res = fit.fit_sweep(m, docs, held, [S], lams)
    r = res[S]
    assert r["rows"] == 1143 and r["lam"] == fit.best_lambda(mine, lams)
    x = torch.randn(10, 256, device=dev).to(torch.bfloat16)
    w, b = maps[r["lam"]][3]
    torch.testing.assert_close(r["projector"](3, x).float(), (x.float() @ w.float().T + b.float()), rtol=2e-2, atol=2e-2)


def test_hybrid_selection_matches_the_oracle(dev):
    """lambda selection on a Qwen3.5-style hybrid (3 GDN : 1 attention, the golden workload of
    tests/golden/q35.py): GDN layers score their pre-conv q / k / v and [b | a] reads, the attention layer its
    k-normed K and V. Device capture, fit and scores against the oracle's scores of the same maps over its own
    bf16 forward (2e-4), the same chosen lambda, fit_sweep end to end; and the scores of the golden maps against
    the ones the reference computed in fp32 (tests/golden/finish_q35.npz, 2e-3: bf16 against fp32 forwards)."""
    import sys
    from pathlib import Path
    import numpy as np
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import q35
    from rfill import fit
    from rfill.model import FillModel
    cfg, t = q35.CONFIG, q35.tensors()
    m = FillModel(cfg, t, dev)
    S = q35.SPLIT
    docs, held = _docs([400, 260, 333, 150], 15, q35.VOCAB), _docs([200, 333], 16, q35.VOCAB)
    lams = (1e-4, 1e-2, 1.0)
    cap = fit.Capture(m, [S])
    for ids in docs:
        cap.add_document(ids)
    maps = fit.fit_maps(cap.state(S, device=dev), lams, device=dev)
    mine = fit.read_scores(m, held, S, maps)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    cpu_maps = {lam: {i: (w.cpu(), b.cpu()) for i, (w, b) in per.items()} for lam, per in maps.items()}
    want = OF.read_scores(om, held, S, cpu_maps)
    worst = max(abs(mine[c][i] - want[c][i]) for c in want for i in want[c])
    print("hybrid scores (device / oracle):", {c: [(round(mine[c][i], 5), round(want[c][i], 5)) for i in mine[c]]
                                              for c in mine}, f"worst {worst:.1e}")
    assert worst < SCORE_TOL
    assert abs(mine["identity"][S] - 1.0) < 1e-6
    mean = {c: sum(v.values()) / len(v) for c, v in want.items()}
    top = sorted((mean[lam] for lam in lams), reverse=True)
    if top[0] - top[1] > 2 * SCORE_TOL:
        assert fit.best_lambda(mine, lams) == OF.best_lambda(want, lams)
    res = fit.fit_sweep(m, docs, held, [S], lams)
    assert res[S]["lam"] == fit.best_lambda(mine, lams) and res[S]["rows"] == 1143
    gold = np.load(q35.FIXTURE)
    gm = {"g": {i: (w.to(dev, torch.bfloat16), b.to(dev, torch.bfloat16)) for i, (w, b) in q35.maps().items()}}
    got = fit.read_scores(m, [q35.held_ids()], S, gm)
    errs = {(c, i): abs(got[c][i] - float(gold[f"score_{'proj' if c == 'g' else 'identity'}_{i}"]))
            for c in got for i in got[c]}
    print("golden scores:", {k: round(v, 6) for k, v in errs.items()})
    assert max(errs.values()) < 2e-3


def test_capture_refuses(dev):
    from rfill import fit
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=3)
    m = FillModel(cfg, t, dev)
    for bad in ([0], [3], []):
        with pytest.raises(ValueError, match="splits"):
            fit.Capture(m, bad)
    with pytest.raises(ValueError, match="block"):
        fit.Capture(m, [1], block=100)
    cap = fit.Capture(m, [1])
    with pytest.raises(ValueError, match="empty"):
        cap.add_document(torch.zeros(0, dtype=torch.int64))
    with pytest.raises(ValueError, match="token ids"):
        cap.add_document(torch.tensor([1, 64]))
    with pytest.raises(ValueError, match="no documents"):
        cap.state(1)
