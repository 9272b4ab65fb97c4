"""GPU parity at the Qwen3-8B shape (hidden 4096, 32 query / 8 KV heads of 128, q_norm and k_norm, RoPE
theta 1e6; the prompt-length sweep of the Qwen3-8B configuration): three late layers (split 18) filled through
ridge maps I + 0.02 N(0, 1/H), with 1 % of the filled rows exact and run through their full layers
(fill_late, as finish() runs them), at a 32768-row prompt (P = 28672, 287 exact rows) and at the sweep's
largest, 122880 rows (P = 118784, 1188 exact rows).

Checked per late layer, on the CPU oracle's bf16 restatement:
  * cache placement: slots >= P keep a sentinel pattern; every value is finite; the exact rows' slots hold
    the K / V of their own inputs: the cache equals, bit for bit, the unsplit device fill of the projected
    rows with each exact row's slot (slot = position) then overwritten by the K / V of its own input
    (FillModel.rows_over_fill over that fill);
  * K / V values of sampled filled rows and of the exact rows against the oracle's kv() of the same inputs;
  * the exact rows' layer outputs (their next layer's inputs) against the oracle's queries, attention over
    the device's filled cache, o_proj and MLP, and a positive control: the projected rows' K at the exact
    slots differs from the exact inputs' by far more than the bar.
Bar: 1e-2 relative Frobenius (the bf16 path's bar)."""
import pytest
import torch
import torch.nn.functional as F

from fill_cases import rel_err
from oracle import model as OM
from oracle import ops as OO

pytestmark = pytest.mark.gpu
TOL = 1e-2
SPLIT, TAIL, N_SAMPLE = 18, 4096, 384
SENTINEL = 0x7F7F                      # a bf16 bit pattern (3.4e38) no fill writes


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def cfg3():
    from rfill import synth
    return dict(synth.QWEN3_8B, num_hidden_layers=SPLIT + 3)


def run_c3(dev, n_rows):
    """The device fill with exact rows; returns everything the checks read (CPU copies of the small parts)."""
    from rfill import synth
    from rfill.kva import Arm, Projector, fill_late
    from rfill.model import FillModel
    cfg = cfg3()
    w = synth.dense_fill(cfg, SPLIT, n_rows, TAIL, device=dev, exact_frac=0.01, full=True)
    P, rows = w["P"], w["rows"]
    model = FillModel(cfg, w["tensors"], dev, layers=w["layers"])
    proj = Projector(SPLIT, w["maps"], w["biases"])
    arm = Arm("ridgefill", split=SPLIT, tail=TAIL, fill="proj", projector=proj)
    cache = model.new_cache()
    for i in w["layers"]:                               # sentinel in every slot, including those >= P
        model.reserve(cache[i], P, model.n_kv, model.head_dim, dev)
        cache[i]["kbuf"].view(torch.int16).fill_(SENTINEL)
        cache[i]["vbuf"].view(torch.int16).fill_(SENTINEL)
    ri = {}
    print(f"[c3] fill_late N={n_rows} P={P} exact={len(rows)}", flush=True)
    cache, P_got = fill_late(model, w["h_split"], arm, exact_rows=rows, cache=cache, row_inputs=ri)
    torch.cuda.synchronize()
    assert P_got == P
    return cfg, w, model, proj, cache, ri


def check_layers(dev, cfg, w, model, proj, cache, ri, out_rows, bitwise_layers=()):
    from rfill import ops
    P, rows = w["P"], w["rows"]
    rows_c = rows.cpu()
    om = OM.OracleModel(cfg, {k: v.cpu() for k, v in w["tensors"].items()}, dtype=torch.bfloat16, layers=w["layers"])
    g = torch.Generator().manual_seed(19)
    filled = torch.ones(P, dtype=torch.bool)
    filled[rows_c] = False                                # rows filled from the projection (not exact rows)
    cand = torch.cat((torch.tensor([0, 1, P - 1]), torch.randperm(P, generator=g)[:2 * N_SAMPLE]))
    cand = cand[filled[cand]]
    sample = torch.unique(cand[:N_SAMPLE + 3])
    b_s = w["h_split"][sample.to(dev)].cpu()
    worst = {"sample": 0.0, "exact": 0.0, "out": 0.0}
    assert torch.equal(ri[SPLIT].cpu(), w["h_split"][rows].cpu())        # the rows enter with h_split[R]
    for i in w["layers"]:
        c = cache[i]
        assert c["n"] == P
        for part in ("kbuf", "vbuf"):
            tail = c[part][:, P:]
            assert bool((tail.view(torch.int16) == SENTINEL).all()), f"layer {i} {part}: a slot >= P was written"
            assert bool(torch.isfinite(c[part][:, :P]).all()), f"layer {i} {part}: non-finite values"
        W, B = proj.W[i].cpu(), proj.b[i].cpu()
        ln1 = om.W[i]["ln1"]
        k_s, v_s = om.kv(i, om.in_norm(F.linear(b_s, W, B), ln1), sample)
        worst["sample"] = max(worst["sample"], rel_err(c["k"][:, sample.to(dev)], k_s),
                              rel_err(c["v"][:, sample.to(dev)], v_s))
        hri = ri[i].cpu()
        xn_r = om.in_norm(hri, ln1)
        k_r, v_r = om.kv(i, xn_r, rows_c)
        ke = rel_err(c["k"][:, rows], k_r)
        worst["exact"] = max(worst["exact"], ke, rel_err(c["v"][:, rows], v_r))
        if i > SPLIT:                                   # positive control: the projected rows' K differs
            k_p, _ = om.kv(i, om.in_norm(F.linear(w["h_split"][rows].cpu(), W, B), ln1), rows_c)
            assert rel_err(k_p, k_r) > 10 * TOL and ke < TOL
        if i in bitwise_layers:                         # placement: bit-exact against fill + the rows' overwrite
            pos = torch.arange(P, device=dev)
            x = proj(i, w["h_split"][:P])
            ref = model.new_cache()
            model.reserve(ref[i], P, model.n_kv, model.head_dim, dev)
            lw = model.W[i]
            cs = model.rope_table(pos)
            ops.norm_kv_write(x, ops.row_ssq(x), model.eps, lw["wkv"], model.n_kv, model.head_dim, lw.get("k_norm"),
                              model.knorm_kind, cs, ref[i]["kbuf"], ref[i]["vbuf"], 0)
            model.commit(ref[i], P)
            model.rows_over_fill(i, ri[i], ops.row_ssq(ri[i]), pos, rows, ref, cs, full=i != w["layers"][-1],
                                 rows_max=P - 1)
            torch.cuda.synchronize()
            assert torch.equal(ref[i]["k"].view(torch.int16), c["k"].view(torch.int16))
            assert torch.equal(ref[i]["v"].view(torch.int16), c["v"].view(torch.int16))
            del ref, x
        if i + 1 in ri:                                  # the rows' layer output = their next layer's input
            sel = out_rows if out_rows is not None else torch.arange(len(rows_c))
            pos_r = rows_c[sel]
            q, _ = om.queries(i, xn_r[sel], pos_r)
            kc, vc = c["k"][:, :P].cpu(), c["v"][:, :P].cpu()
            o = OO.attend_at(q, kc, vc, om.scale, pos_r)
            want = om.mlp(i, hri[sel] + F.linear(o, om.W[i]["o"]))
            worst["out"] = max(worst["out"], rel_err(ri[i + 1][sel.to(dev)], want))
        print(f"[c3] layer {i}: sampled K/V {worst['sample']:.2e}, exact-row K/V {worst['exact']:.2e}, "
              f"row outputs {worst['out']:.2e}", flush=True)
    del om
    assert max(worst.values()) < TOL, worst


def test_exact_rows_c3_32k(dev):
    cfg, w, model, proj, cache, ri = run_c3(dev, 32768)
    assert len(w["rows"]) == 287
    check_layers(dev, cfg, w, model, proj, cache, ri, None, bitwise_layers=(SPLIT, SPLIT + 1))


def test_exact_rows_c3_122880(dev):
    """The sweep's largest prompt: P = 118784 (the widest row, slot and position ranges every fill kernel
    indexes), 1188 exact rows; row outputs checked on the 96 rows nearest P (the longest attention)."""
    cfg, w, model, proj, cache, ri = run_c3(dev, 122880)
    n = len(w["rows"])
    assert n == 1188 and w["P"] == 118784
    check_layers(dev, cfg, w, model, proj, cache, ri, torch.arange(n - 96, n))
