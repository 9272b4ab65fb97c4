"""GPU parity at the Qwen3.5-shaped hybrid's own widths (hidden 2048; GDN 16 key / 32 value heads of 128)
with the architecture's own gate initialisation (rfill.synth.gdn_layer_weights: A_log = log U(0, 16),
dt_bias = 1, so per-row decays reach e^-16): the Gated DeltaNet fill over all 28672 filled rows (448 chunk
steps in 4 workspace passes) and the exact GDN layer's delta-rule outputs (rf_gdn_forward: prep, scan and
the output kernel) over a 4096-row tail, each against the oracle's chunked rule fed the device's own
in-projection rows. Bars: the conv state bit-exact; the recurrent state and the outputs within 1e-2
relative Frobenius (the bf16 path's bar; the measured errors are printed)."""
import pytest
import torch

from fill_cases import rel_err
from oracle import model as OM

pytestmark = pytest.mark.gpu
TOL = 1e-2
LAYER = 24


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.fixture(scope="module")
def c4(dev):
    from rfill import synth
    from rfill.model import FillModel
    cfg = synth.QWEN35_HYBRID
    t = synth.gdn_layer_weights(cfg, LAYER)
    m = FillModel(cfg, t, dev, layers=[LAYER])
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16, layers=[LAYER])
    return cfg, m, om


def _split(pre, om):
    C = 2 * om.nk * om.dk + om.nv * om.dv
    return pre[:, :C], pre[:, C:C + om.nv], pre[:, C + om.nv:C + 2 * om.nv]


def test_gdn_fill_full_depth_c4(dev, c4):
    """FillModel.fill of one C4 GDN layer over 28672 rows from zero state vs the oracle's conv + gates +
    chunked rule on the same in-projection rows."""
    from rfill import ops, synth
    cfg, m, om = c4
    P, H = 28672, cfg["hidden_size"]
    x = synth.hidden_states(P, H, device=dev)
    cache = m.new_cache()
    m.fill(LAYER, x, torch.arange(P, device=dev), cache)
    pre = ops.norm_linear(x, ops.row_ssq(x), m.eps, m.W[LAYER]["w_in"])      # the rows the fill consumed
    torch.cuda.synchronize()
    oc = om.new_cache()
    om.gdn_core(LAYER, *_split(pre.cpu(), om), oc, False)
    err = rel_err(cache[LAYER]["rec"], oc[LAYER]["rec"])
    print(f"C4 GDN fill, {P} rows: recurrent state rel err {err:.2e}, |S| {float(oc[LAYER]['rec'].norm()):.3g}")
    assert cache[LAYER]["len"] == P
    assert torch.equal(cache[LAYER]["conv"].cpu(), oc[LAYER]["conv"])
    assert bool(torch.isfinite(cache[LAYER]["rec"]).all()) and err < TOL


def test_gdn_forward_outputs_c4(dev, c4):
    """rf_gdn_forward over a 4096-row tail (64 chunks x 32 value heads: k_gdn_out at the hybrid's shape)
    continuing a 2048-row filled state and conv state, vs the oracle's chunked rule with outputs from the
    same starting states; the final state bit-identical to rf_gdn_fill's over the same rows."""
    from rfill import ops, synth
    cfg, m, om = c4
    H, nk, nv = cfg["hidden_size"], m.nk, m.nv
    w = m.W[LAYER]
    x = synth.hidden_states(2048 + 4096, H, device=dev, seed_rows=70)
    pre = ops.norm_linear(x, ops.row_ssq(x), m.eps, w["w_in"])
    st = torch.zeros(nv, 128, 128, dtype=torch.float32, device=dev)
    conv = ops.gdn_fill(pre[:2048], nk, nv, 128, 128, w["conv"], None, w["a_log"], w["dt_bias"], st)
    st0, conv0 = st.clone(), conv.clone()
    out, conv1 = ops.gdn_forward(pre[2048:], nk, nv, 128, 128, w["conv"], conv, w["a_log"], w["dt_bias"], st)
    st_fill = st0.clone()
    conv_fill = ops.gdn_fill(pre[2048:], nk, nv, 128, 128, w["conv"], conv0, w["a_log"], w["dt_bias"], st_fill)
    torch.cuda.synchronize()
    oc = om.new_cache()
    oc[LAYER] = {"rec": st0.cpu(), "conv": conv0.cpu()}
    want, _ = om.gdn_core(LAYER, *_split(pre[2048:].cpu(), om), oc, True)
    want = want.transpose(0, 1).reshape(4096, nv * 128)
    err = rel_err(out, want)
    es = rel_err(st, oc[LAYER]["rec"])
    worst_head = max(rel_err(out[:, 128 * j:128 * (j + 1)], want[:, 128 * j:128 * (j + 1)]) for j in range(nv))
    print(f"C4 GDN forward, 4096 rows x {nv} heads: outputs rel err {err:.2e} (worst head {worst_head:.2e}), "
          f"state {es:.2e}")
    assert err < TOL and worst_head < TOL and es < TOL
    assert torch.equal(st, st_fill) and torch.equal(conv1, conv_fill)
