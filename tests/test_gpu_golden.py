"""The device path against the golden vectors of the reference implementation
(tests/golden/finish_c1.npz, written by tests/golden/make_golden.py) on the tiny Llama-style workload:

  * fill_late (bf16) for the ridgefill arm, the identity arm and the ridgefill arm with 18 exact rows
    (their late-layer inputs taken from the fixture): the filled cache rows [0, P) against the
    reference's fp32 caches, relative Frobenius error <= 1e-2 (the bf16 bar), and n / slots exact;
  * finish() (fill, exact tail, logits) for the same three arms: the tail logits (probe projections, the
    last row, argmax) and every cache slot including the tail's, against the reference's finish();
  * the device fit (RidgeStats + RidgeFit on the GPU) from the calibration rows in bf16 against the
    reference's fp32-row maps (1e-2: the rows are rounded to bf16 before the products).

The split-layer rows and the maps fed to the fill come from the oracle, which tests/test_golden_c1.py
pins to the same fixture at 1e-4.
"""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import c1  # noqa: E402

from test_golden_c1 import oracle_run, rel  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(c1.FIXTURE))


@pytest.fixture(scope="module")
def run():
    return oracle_run()


@pytest.mark.parametrize("name", ["proj", "identity", "exact", "exact_computed"])
def test_fill_late_matches_reference(dev, gold, run, name):
    from rfill.kva import Arm, Projector, fill_late
    from rfill.model import FillModel
    S, L = c1.SPLIT, c1.CONFIG["num_hidden_layers"]
    late = list(range(S, L))
    model = FillModel(c1.CONFIG, c1.tensors(), dev, layers=late)
    W = {i: w for i, (w, _) in run["maps"].items()}
    B = {i: b for i, (_, b) in run["maps"].items()}
    fill = "identity" if name == "identity" else "proj"
    arm = Arm(name, split=S, tail=c1.TAIL, fill=fill, projector=Projector(S, W, B) if fill == "proj" else None)
    h_split = run["hs"][S].to(dev, torch.bfloat16)
    rows = hr = None
    row_inputs = {}
    if name == "exact":              # the rows' inputs given (the reference's row_inputs)
        rows = c1.exact_rows()
        hr = {i: torch.from_numpy(gold[f"exact_hr_{i}"]).to(dev, torch.bfloat16) for i in late}
    elif name == "exact_computed":   # the rows run through every late layer on the device (layer_rows)
        rows = c1.exact_rows()
    cache, P = fill_late(model, h_split, arm, exact_rows=rows, hr=hr, row_inputs=row_inputs)
    torch.cuda.synchronize()
    gname = "exact" if name == "exact_computed" else name
    assert P == int(gold[f"{gname}_P"])
    if name == "exact_computed":
        for i in late:
            err = rel(row_inputs[i].double().cpu().numpy(), gold[f"exact_hr_{i}"])
            print(f"exact rows' input to layer {i}: rel err vs the reference {err:.2e}")
            assert err < TOL, (i, err)
    u = c1.probes(102, 64)
    worst = 0.0
    for i in late:
        assert cache[i]["n"] == P
        for part in ("k", "v"):
            got = (cache[i][part].double().cpu() @ u).numpy()          # [Hkv, P]
            want = gold[f"{gname}_{part}_u_{i}"][:, :P]
            err = rel(got, want)
            worst = max(worst, err)
            assert err < TOL, (i, part, err)
            # the rows the fixture keeps in full: slots 0, 1, P - 1
            full = cache[i][part][:, [0, 1, P - 1]].double().cpu().numpy()
            assert rel(full, gold[f"{gname}_{part}_rows_{i}"][:, :3]) < TOL
    print(f"{name}: worst K/V rel err vs the reference {worst:.2e}")


def test_device_fit_matches_reference(dev, gold, run):
    from rfill import ridge
    S, L = c1.SPLIT, c1.CONFIG["num_hidden_layers"]
    late = list(range(S, L))
    cal = run["calibration"]
    st = ridge.RidgeStats(S, late, c1.CONFIG["hidden_size"], device=dev)
    st.add(cal[S].to(dev, torch.bfloat16), {i: cal[i].to(dev, torch.bfloat16) for i in late})
    fit = ridge.RidgeFit(st.state(device=dev), device=dev)
    assert st.n == c1.N_CAL
    u, v = c1.probes(100, 256), c1.probes(101, 256)
    worst = 0.0
    for i in late:
        w, b = fit.layer(i, (c1.LAM,))[c1.LAM]
        w = w.double().cpu()
        for got, key in ((w @ u, f"w_u_{i}"), (w.T @ v, f"w_tv_{i}"), (b.double().cpu(), f"bias_{i}")):
            err = rel(got.numpy(), gold[key])
            worst = max(worst, err)
            assert err < TOL, (key, err)
    print(f"device fit from bf16 rows: worst map rel err vs the reference {worst:.2e}")


@pytest.mark.parametrize("name", ["proj", "identity", "exact"])
def test_finish_matches_reference(dev, gold, run, name):
    """The whole late stack on the device -- the fill, the exact rows through their layers, the 256-row
    exact tail through every late layer and the logits of the last 256 rows -- against the reference's
    own finish() on the same model and split-layer rows."""
    from rfill.kva import Arm, Projector, finish
    from rfill.model import FillModel
    S, L = c1.SPLIT, c1.CONFIG["num_hidden_layers"]
    late = list(range(S, L))
    model = FillModel(c1.CONFIG, c1.tensors(), dev, layers=late)
    W = {i: w for i, (w, _) in run["maps"].items()}
    B = {i: b for i, (_, b) in run["maps"].items()}
    fill = "identity" if name == "identity" else "proj"
    arm = Arm(name, split=S, tail=c1.TAIL, fill=fill, projector=Projector(S, W, B) if fill == "proj" else None)
    rows = c1.exact_rows() if name == "exact" else None
    logits, cache, P = finish(model, c1.prompt_ids(), run["hs"][S], None, arm, c1.KEEP, exact_rows=rows)
    torch.cuda.synchronize()
    assert P == int(gold[f"{name}_P"])
    lg = logits.double().cpu()
    el = rel(lg.numpy() @ c1.probes(103, 1024, 4).numpy(), gold[f"{name}_logits_u"])
    elast = rel(lg[-1].numpy(), gold[f"{name}_logits_last"])
    agree = float((lg.argmax(-1).numpy() == gold[f"{name}_argmax"]).mean())
    u = c1.probes(102, 64)
    worst = 0.0
    for i in late:
        assert cache[i]["n"] == int(gold[f"{name}_n_{i}"]) == c1.N_PROMPT
        for part in ("k", "v"):
            got = (cache[i][part].double().cpu() @ u).numpy()
            worst = max(worst, rel(got, gold[f"{name}_{part}_u_{i}"]))
            assert rel(got[:, P:], gold[f"{name}_{part}_u_{i}"][:, P:]) < TOL      # the tail's own slots
    print(f"{name}: tail logits rel err {el:.2e} (last row {elast:.2e}), argmax agreement {agree:.3f}, "
          f"worst K/V {worst:.2e}")
    assert el < TOL and elast < TOL and worst < TOL and agree > 0.9
