"""GPU parity of the Qwen3.5 exact layers (code/kva/model.py:386-556): the GDN mixing with outputs
(rf_gdn_forward) against the oracle's chunked delta rule, its state bit-identical to the fill's; the
output gate and the gated output norm against the oracle's bf16 formulas; the gated attention layer
(head_dim 256, partial RoPE) and the GDN layer through FillModel.layer / layer_rows against the oracle;
a hybrid model's exact forward and the capture sums over it. Bars: 1e-2 relative Frobenius for the bf16
paths; 2e-2 for a layer output's update (output - input: both sides round the output to bf16, 2^-9 of |out|,
and the update is a fraction of |out|, so that rounding alone is several 1e-3 of the update) and for the
inputs of layers past the first of the hybrid's exact forward (each carries the earlier layers' differences);
1e-5 for the capture sums."""
import pytest
import torch
import torch.nn.functional as F

from fill_cases import case, hybrid_config, hybrid_tensors, inputs, rel_err
from oracle import model as OM
from oracle import ops as OO
from oracle import ridge as oridge

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.fixture(scope="module")
def hybrid():
    cfg = hybrid_config(["gdn", "gdn", "gdn", "attn"])
    return cfg, hybrid_tensors(cfg, seed=3)


def _oracle_out(om, i, pre_full, cache):
    """The oracle's delta-rule outputs [n, nv dv] (bf16) for the in-projection rows pre_full."""
    C = 2 * om.nk * om.dk + om.nv * om.dv
    pre, b, a = pre_full[:, :C], pre_full[:, C:C + om.nv], pre_full[:, C + om.nv:C + 2 * om.nv]
    out, _ = om.gdn_core(i, pre, b, a, cache, True)
    return out.transpose(0, 1).reshape(pre.shape[0], -1)


def test_gdn_forward_matches_oracle(dev, hybrid):
    """Two calls (300 rows, then 130 continuing the conv and recurrent states): outputs against the
    oracle, states bit-identical to rf_gdn_fill's, and a one-chunk workspace (many passes) giving the same bits."""
    from rfill import ops
    from rfill.model import FillModel
    cfg, t = hybrid
    m = FillModel(cfg, t, dev)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    w = m.W[0]
    x = inputs(430, cfg["hidden_size"], seed=41)
    pre = ops.norm_linear(x.to(dev), ops.row_ssq(x.to(dev)), m.eps, w["w_in"])
    pre_c = pre.cpu()
    oc = om.new_cache()
    st = torch.zeros(m.nv, 128, 128, dtype=torch.float32, device=dev)
    st_fill = st.clone()
    conv = conv_fill = None
    outs = []
    for r0, r1 in ((0, 300), (300, 430)):
        o, conv_new = ops.gdn_forward(pre[r0:r1], m.nk, m.nv, 128, 128, w["conv"], conv, w["a_log"], w["dt_bias"], st)
        conv_fill = ops.gdn_fill(pre[r0:r1], m.nk, m.nv, 128, 128, w["conv"], conv_fill, w["a_log"], w["dt_bias"],
                                 st_fill)
        conv = conv_new
        outs.append(o)
        want = _oracle_out(om, 0, pre_c[r0:r1], oc)
        err = rel_err(o, want)
        print(f"rows {r0}..{r1}: out rel err {err:.2e}, state vs oracle {rel_err(st, oc[0]['rec']):.2e}")
        assert err < TOL
    torch.cuda.synchronize()
    assert torch.equal(st, st_fill) and torch.equal(conv, conv_fill)
    # one chunk per pass
    st2 = torch.zeros_like(st)
    ws = torch.empty(ops.gdn_forward_workspace_bytes(0, m.nk, m.nv), dtype=torch.uint8, device=dev)
    o2, _ = ops.gdn_forward(pre[:300], m.nk, m.nv, 128, 128, w["conv"], None, w["a_log"], w["dt_bias"], st2,
                            workspace=ws)
    st3 = torch.zeros_like(st)
    o3, _ = ops.gdn_forward(pre[:300], m.nk, m.nv, 128, 128, w["conv"], None, w["a_log"], w["dt_bias"], st3)
    torch.cuda.synchronize()
    assert torch.equal(o2, o3) and torch.equal(o3, outs[0]) and torch.equal(st2, st3)


def test_gate_and_gated_norm_kernels(dev):
    from rfill import ops
    g = torch.Generator().manual_seed(42)
    o = (torch.randn(37, 512, generator=g)).to(torch.bfloat16)
    gt = (2 * torch.randn(37, 512, generator=g)).to(torch.bfloat16)
    got = ops.sigmoid_mul(o.to(dev), gt.to(dev)).cpu()
    want = o * torch.sigmoid(gt)
    diff = (got.float() - want.float()).abs()
    ulp = want.float().abs() * 2.0 ** -7
    assert bool((diff <= ulp + 1e-30).all()) and float((got != want).float().mean()) < 0.01
    x = (torch.randn(37, 4 * 128, generator=g)).to(torch.bfloat16)
    z = (torch.randn(37, 4 * 128, generator=g)).to(torch.bfloat16)
    wt = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    got = ops.gated_rms_norm(x.to(dev), z.to(dev), wt.to(dev), 4, 128, 1e-6).cpu()
    want = OO.rms_norm_gated(x.view(37, 4, 128), z.view(37, 4, 128), wt, 1e-6).reshape(37, -1)
    diff = (got.float() - want.float()).abs()
    ulp = want.float().abs() * 2.0 ** -7
    print(f"gated norm: {float((got != want).float().mean()):.4f} of values differ")
    assert bool((diff <= ulp + 1e-30).all()) and float((got != want).float().mean()) < 0.01


def _layer_case(name):
    if name == "qwen35_attn":
        return case("qwen35_attn")
    cfg = hybrid_config(["gdn"])
    return cfg, hybrid_tensors(cfg, seed=5)


@pytest.mark.parametrize("name", ["qwen35_attn", "gdn"])
def test_layer_matches_oracle(dev, name):
    """P filled rows, then T rows through the exact layer (the tail): output and the layer's cache state."""
    from rfill.model import FillModel
    cfg, t = _layer_case(name)
    P, T, H = 700, 200, cfg["hidden_size"]
    x, h = inputs(P, H, seed=43), inputs(T, H, seed=44)
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
    err = rel_err(got, want)
    ed = rel_err(got.cpu().float() - h.float(), want.float() - h.float())
    es = rel_err(ssq.sum(1), got.float().pow(2).sum(1))
    if name == "gdn":
        ec = rel_err(c[0]["rec"], oc[0]["rec"])
        assert c[0]["len"] == P + T
    else:
        ec = rel_err(c[0]["k"], oc[0]["k"])
        assert c[0]["n"] == P + T
    print(f"{name}: out {err:.2e}, update {ed:.2e}, cache {ec:.2e}, ssq {es:.1e}")
    assert err < TOL and ed < 2 * TOL and ec < TOL and es < 1e-5


@pytest.mark.parametrize("name", ["qwen35_attn", "gdn"])
def test_layer_rows_matches_oracle(dev, name):
    from rfill.model import FillModel
    cfg, t = _layer_case(name)
    P, H = 600, cfg["hidden_size"]
    x = inputs(P, H, seed=45)
    pos = torch.arange(P)
    rows = torch.tensor([0, 5, 63, 64, 300, 599])
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    want = om.layer_rows(0, x, pos, rows, om.new_cache())
    m = FillModel(cfg, t, dev)
    got = m.layer_rows(0, x.to(dev), pos.to(dev), rows, m.new_cache())
    torch.cuda.synchronize()
    err = rel_err(got, want)
    ed = rel_err(got.cpu().float() - x[rows].float(), want.float() - x[rows].float())
    print(f"{name} rows: out {err:.2e}, update {ed:.2e}")
    assert err < TOL and ed < 2 * TOL


def test_hybrid_forward_and_capture(dev, hybrid):
    """A 4-layer hybrid (3 GDN : 1 attention): every layer input against the oracle's exact forward, and
    the capture sums (split 1) against the oracle's Capture fed the device's own inputs."""
    from rfill import fit
    from rfill.model import FillModel
    cfg, t = hybrid
    g = torch.Generator().manual_seed(46)
    docs = [torch.randint(0, 64, (n,), generator=g) for n in (300, 129)]
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    m = FillModel(cfg, t, dev)
    want, mine = {}, {}
    om.forward_exact(docs[0], hook=lambda i, h: want.__setitem__(i, h))
    m.forward_exact(docs[0], hook=lambda i, h: mine.__setitem__(i, h.clone()))
    torch.cuda.synchronize()
    errs = {i: rel_err(mine[i], want[i]) for i in (1, 2, 3, "final")}
    print("hybrid layer inputs:", {k: f"{v:.2e}" for k, v in errs.items()})
    assert all(e < 2 * TOL for e in errs.values())
    cap = fit.Capture(m, [1], block=256)
    ref = oridge.Capture([1], 4, cfg["hidden_size"])
    for ids in docs:
        cap.add_document(ids)
        got = {}
        m.forward_exact(ids, hook=lambda i, h: got.__setitem__(i, h.float().cpu()) if i != "final" and i >= 1 else None)
        ref.add_document(got)
    a, b = cap.state(1), ref.state(1)
    e = max(rel_err(a["sxx"], b["sxx"]), *(rel_err(a["sxy"][i], b["sxy"][i]) for i in (1, 2, 3)))
    print(f"hybrid capture sums: {e:.1e}")
    assert a["n"] == 429 and e < 1e-5


@pytest.mark.parametrize("exact", [False, True])
def test_hybrid_finish_matches_oracle(dev, exact):
    """finish() on an 8-layer hybrid (GDN, GDN, GDN, attention, twice), split 4: the fill of the late
    layers (with exact rows through their GDN and attention layers, or none), the terminal-state
    corrections st on the late GDN layers, the 192-row exact tail through every late layer, tail logits."""
    from oracle import kva as OK
    from rfill.kva import Arm, Projector, finish
    from rfill.model import FillModel
    cfg = hybrid_config(["gdn", "gdn", "gdn", "attn"] * 2)
    t = hybrid_tensors(cfg, seed=7)
    N, tail, split, keep = 900, 192, 4, 64
    P, H = N - tail, cfg["hidden_size"]
    h = inputs(N, H, seed=47)
    g = torch.Generator().manual_seed(48)
    W = {i: (torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16) for i in range(split, 8)}
    B = {i: (1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for i in range(split, 8)}
    st = {i: 0.01 * torch.randn(4, 128, 128, generator=g) for i in (4, 5, 6)}
    rows = torch.randperm(P, generator=g)[:12].sort().values if exact else None
    m = FillModel(cfg, t, dev)
    arm = Arm("ridgefill", split=split, tail=tail, fill="proj", projector=Projector(split, W, B),
              st={i: s.to(dev) for i, s in st.items()})
    logits, cache, P_got = finish(m, torch.zeros(N, dtype=torch.long), h.to(dev), None, arm, keep, exact_rows=rows)
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oarm = OK.Arm("ridgefill", split=split, tail=tail, fill="proj", projector=OK.Projector(split, W, B), st=st)
    want, oc, P_want = OK.finish(om, torch.zeros(N, dtype=torch.long), h, om.new_cache(), oarm, keep, exact_rows=rows)
    assert P_got == P_want == P
    el = rel_err(logits, want)
    es = max(rel_err(cache[i]["rec"], oc[i]["rec"]) for i in (4, 5, 6))
    ek = max(rel_err(cache[7][part], oc[7][part]) for part in ("k", "v"))
    agree = float((logits.argmax(-1).cpu() == want.argmax(-1)).float().mean())
    print(f"hybrid finish (exact rows: {exact}): logits {el:.2e}, GDN states {es:.2e}, K/V {ek:.2e}, argmax {agree:.3f}")
    assert el < TOL and es < TOL and ek < TOL and agree > 0.9
