"""GPU parity of the Gated DeltaNet fill (rf_norm_linear + rf_gdn_fill) against the CPU oracle, whose GDN
math is pinned to transformers' Qwen3.5 (tests/test_oracle_model.py). Bars: the conv state is a copy of
pre-conv rows, bit-exact; with the oracle's own in-projection rows as input the recurrent state agrees
to fp32 rounding (<= 1e-4 relative Frobenius; the products run on bf16 MFMA with fp32 operands split
into hi + lo bf16 halves); through the whole bf16 fill path <= 1e-2."""
import pytest
import torch

from fill_cases import gdn_config, gdn_tensors, inputs, rel_err
from oracle import model as OM

pytestmark = pytest.mark.gpu
STATE_TOL = 1e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch.device("cuda")


def _pre_rows(om, x):
    """The oracle's in-projection rows [P, C + 2 nv] (q | k | v | b | a), bf16, as rf_gdn_fill reads them."""
    pre, b, a = om.gdn_inputs(0, om.in_norm(x, om.W[0]["ln1"]))
    return torch.cat((pre, b, a), 1)


@pytest.mark.parametrize("P", [1000, 64, 3])
def test_recurrence_matches_oracle_given_the_same_rows(dev, P):
    from rfill import ops
    cfg = gdn_config()
    t = gdn_tensors(cfg)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    x = inputs(P, cfg["hidden_size"], seed=21)
    c = om.new_cache()
    om.fill(0, x, torch.arange(P), c)
    rows = _pre_rows(om, x).to(dev)
    w = om.W[0]
    state = torch.zeros(4, 128, 128, dtype=torch.float32, device=dev)
    conv = ops.gdn_fill(rows, 2, 4, 128, 128, w["conv"].to(dev).contiguous(), None, w["A_log"].to(dev),
                        w["dt_bias"].to(dev), state)
    torch.cuda.synchronize()
    err = rel_err(state, c[0]["rec"])
    print(f"P {P}: recurrent state rel err {err:.2e}")
    assert err < 1e-4
    assert torch.equal(conv.cpu(), c[0]["conv"])


def test_workspace_passes_are_bitwise_equal(dev):
    """A workspace of 1 or 3 chunks (several prep / scan passes) gives the single pass's bits."""
    from rfill import ops
    cfg = gdn_config()
    t = gdn_tensors(cfg, seed=4)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    x = inputs(700, cfg["hidden_size"], seed=24)
    rows = _pre_rows(om, x).to(dev)
    w = om.W[0]
    args = (w["conv"].to(dev).contiguous(), None, w["A_log"].to(dev), w["dt_bias"].to(dev))
    out = {}
    for chunks in (None, 1, 3):
        st = torch.zeros(4, 128, 128, dtype=torch.float32, device=dev)
        ws = None
        if chunks:
            ws = torch.empty(chunks * ops.gdn_workspace_bytes(0, 2, 4), dtype=torch.uint8, device=dev)
        conv = ops.gdn_fill(rows, 2, 4, 128, 128, *args, st, ws)
        out[chunks] = (st, conv)
    torch.cuda.synchronize()
    for chunks in (1, 3):
        assert torch.equal(out[chunks][0], out[None][0]) and torch.equal(out[chunks][1], out[None][1])
    with pytest.raises(ValueError):
        ops.gdn_fill(rows, 2, 4, 128, 128, *args, out[None][0],
                     torch.empty(ops.gdn_workspace_bytes(0, 2, 4) - 16, dtype=torch.uint8, device=dev))


@pytest.mark.parametrize("chunks", [None, 3])
def test_batched_layers_are_bitwise_their_single_fills(dev, chunks):
    """rf_gdn_fill_batch over two layers (different weights, rows, carried conv and recurrent states) against
    rf_gdn_fill of each alone: every state and conv state bit for bit, in one pass and in several (a workspace
    of 3 chunks per layer)."""
    from rfill import ops
    cfg = gdn_config()
    jobs, single = [], []
    for seed in (5, 6):
        om = OM.OracleModel(cfg, gdn_tensors(cfg, seed=seed), dtype=torch.bfloat16)
        rows = _pre_rows(om, inputs(900, cfg["hidden_size"], seed=30 + seed)).to(dev)
        w = om.W[0]
        g = torch.Generator().manual_seed(seed)
        st0 = (0.1 * torch.randn(4, 128, 128, generator=g)).to(dev)
        conv_in = torch.randn(3, 2 * 2 * 128 + 4 * 128, generator=g).to(torch.bfloat16).to(dev)   # [3, C]
        args = (w["conv"].to(dev).contiguous(), conv_in, w["A_log"].to(dev), w["dt_bias"].to(dev))
        st = st0.clone()
        conv = ops.gdn_fill(rows, 2, 4, 128, 128, *args, st)
        single.append((st, conv))
        jobs.append((rows, *args, st0.clone()))
    ws = None if chunks is None else torch.empty(2 * chunks * ops.gdn_workspace_bytes(0, 2, 4), dtype=torch.uint8,
                                                 device=dev)
    convs = ops.gdn_fill_batch(jobs, 2, 4, 128, 128, ws)
    torch.cuda.synchronize()
    for (st, conv), job, cb in zip(single, jobs, convs):
        assert torch.equal(job[5], st) and torch.equal(cb, conv)
    with pytest.raises(ValueError, match="share"):
        ops.gdn_fill_batch([jobs[0], jobs[0]], 2, 4, 128, 128)


def test_fill_matches_oracle_and_continues(dev):
    """FillModel.fill (in-projection GEMM + GDN kernel) against the oracle's fill, then a second call
    continuing both states; plus the terminal-state correction st."""
    from rfill.model import FillModel
    cfg = gdn_config()
    t = gdn_tensors(cfg, seed=1)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    m = FillModel(cfg, t, dev)
    x = inputs(1500, cfg["hidden_size"], seed=22)
    oc, mc = om.new_cache(), m.new_cache()
    for a, b in ((0, 1100), (1100, 1500)):
        om.fill(0, x[a:b], torch.arange(a, b), oc)
        m.fill(0, x[a:b].to(dev), torch.arange(a, b, device=dev), mc)
        torch.cuda.synchronize()
        err = rel_err(mc[0]["rec"], oc[0]["rec"])
        conv = rel_err(mc[0]["conv"], oc[0]["conv"])
        print(f"rows [{a}, {b}): state rel err {err:.2e}, conv state rel err {conv:.2e}")
        assert err < STATE_TOL and conv < STATE_TOL and mc[0]["len"] == oc[0]["len"] == b
    st = 0.01 * torch.randn(4, 128, 128, generator=torch.Generator().manual_seed(3))
    before = mc[0]["rec"].clone()
    m2 = m.new_cache()
    m2[0] = dict(mc[0], rec=before.clone())
    m.fill(0, x[:0].to(dev), torch.arange(0, device=dev), m2)          # zero rows: nothing changes
    assert torch.equal(m2[0]["rec"], before)
    one = m.new_cache()
    m.fill(0, x[:200].to(dev), torch.arange(200, device=dev), one, st=st.to(dev))
    ref = om.new_cache()
    om.fill(0, x[:200], torch.arange(200), ref, st=st)
    assert rel_err(one[0]["rec"], ref[0]["rec"]) < STATE_TOL


def test_fill_matches_the_full_projection_bitwise(dev):
    """FillModel.fill projects q for the conv state's last 3 rows only; its states are bit-identical to
    rf_gdn_fill on the whole in-projection, and FillModel.fill_batch over two layers to fill of each."""
    from rfill import ops
    from rfill.model import FillModel
    cfg = gdn_config(layers=2)
    m = FillModel(cfg, gdn_tensors(cfg, seed=7), dev)
    x = inputs(777, cfg["hidden_size"], seed=23).to(dev)
    ssq = ops.row_ssq(x)
    c = m.new_cache()
    m.fill(0, x, None, c, ssq=ssq)
    w = m.W[0]
    pre = ops.norm_linear(x, ssq, m.eps, w["w_in"])
    st = torch.zeros(m.nv, m.dk, m.dv, dtype=torch.float32, device=dev)
    conv = ops.gdn_fill(pre, m.nk, m.nv, m.dk, m.dv, w["conv"], None, w["a_log"], w["dt_bias"], st)
    torch.cuda.synchronize()
    assert torch.equal(c[0]["rec"], st) and torch.equal(c[0]["conv"], conv)
    x2 = inputs(777, cfg["hidden_size"], seed=25).to(dev)
    one, two = m.new_cache(), m.new_cache()
    m.fill(0, x, None, one)
    m.fill(1, x2, None, one)
    m.fill_batch([0, 1], [x, x2], two)
    torch.cuda.synchronize()
    for i in (0, 1):
        assert torch.equal(one[i]["rec"], two[i]["rec"]) and torch.equal(one[i]["conv"], two[i]["conv"])
        assert one[i]["len"] == two[i]["len"] == 777


def test_fill_c4_gdn_layer_shape(dev):
    """One GDN layer at the hybrid config's widths (hidden 2048, 16 key / 32 value heads) over 2048 rows."""
    from rfill.model import FillModel
    cfg = gdn_config(hidden=2048, nk=16, nv=32)
    t = gdn_tensors(cfg, seed=2)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    m = FillModel(cfg, t, dev)
    x = inputs(2048, 2048, seed=23)
    oc, mc = om.new_cache(), m.new_cache()
    om.fill(0, x, torch.arange(2048), oc)
    m.fill(0, x.to(dev), torch.arange(2048, device=dev), mc)
    torch.cuda.synchronize()
    err = rel_err(mc[0]["rec"], oc[0]["rec"])
    print(f"C4 GDN layer: state rel err {err:.2e}")
    assert err < STATE_TOL


def test_fill_checkpoints(dev):
    """fill(..., checkpoint_every=256) over 1100 rows continuing 300 filled rows: the states after 256,
    512, 768 and 1024 rows of the call, keyed by position (300 + t), against the oracle's checkpoints; the
    final state and conv state bit-identical to a fill without checkpoints."""
    from rfill.model import FillModel
    cfg = gdn_config()
    t = gdn_tensors(cfg, seed=4)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    m = FillModel(cfg, t, dev)
    x = inputs(1400, cfg["hidden_size"], seed=23)
    oc, mc, plain = om.new_cache(), m.new_cache(), m.new_cache()
    om.fill(0, x[:300], torch.arange(300), oc)
    for c in (mc, plain):
        m.fill(0, x[:300].to(dev), torch.arange(300, device=dev), c)
    want = om.fill(0, x[300:], torch.arange(300, 1400), oc, checkpoint_every=256)
    got = m.fill(0, x[300:].to(dev), torch.arange(300, 1400, device=dev), mc, checkpoint_every=256)
    m.fill(0, x[300:].to(dev), torch.arange(300, 1400, device=dev), plain)
    torch.cuda.synchronize()
    assert sorted(got) == sorted(want) == [556, 812, 1068, 1324]
    errs = {k: rel_err(got[k], want[k]) for k in got}
    print("checkpoint state rel errs", {k: f"{v:.2e}" for k, v in errs.items()})
    assert all(e < STATE_TOL for e in errs.values())
    assert torch.equal(mc[0]["rec"], plain[0]["rec"]) and torch.equal(mc[0]["conv"], plain[0]["conv"])
    with pytest.raises(ValueError, match="multiple"):
        m.fill(0, x[:64].to(dev), torch.arange(64, device=dev), m.new_cache(), checkpoint_every=100)
