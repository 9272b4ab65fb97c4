"""The oracle against golden vectors written by the reference implementation itself
(tests/golden/finish_c1.npz from tests/golden/make_golden.py): on the tiny Llama-style workload of
tests/golden/c1.py, in fp32 on the CPU,
  * fit_sweep's capture sums (code/scripts/fit_sweep.py:87-166) over one and over two documents
    (the shifts are the FIRST document's means, not the overall means);
  * RidgeFit.layer (code/kva/ridge.py:77-105) at lambda 1e-2: lambda scaled by the centred scatter's
    mean diagonal, bias unpenalised;
  * the composed finish() (code/kva/kva.py:319-460) for the ridgefill arm, the identity arm and the
    ridgefill arm with 18 exact rows: filled K / V caches (placement and values), the exact rows'
    late-layer inputs and the tail logits.
Each group has a positive control: a plausible mistake planted in the oracle's inputs or conventions
(shift = overall mean, lambda on the uncentred scatter, exact rows not scattered) fails the same check.
"""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import c1  # noqa: E402

from oracle import kva as OK  # noqa: E402
from oracle import ridge as OR  # noqa: E402
from oracle.model import OracleModel  # noqa: E402

RTOL = 1e-4


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(c1.FIXTURE))


@pytest.fixture(scope="module")
def run():
    return oracle_run()


def oracle_run():
    """The oracle's capture, fit and three finish runs on the golden workload."""
    torch.manual_seed(0)
    m = OracleModel(c1.CONFIG, c1.tensors(), dtype=torch.float32)
    S, L = c1.SPLIT, m.n_layers

    def capture(docs):
        cap = OR.Capture([S], L, m.hidden)
        for doc in docs:
            got = {}
            m.forward_exact(doc, hook=lambda i, h: got.__setitem__(i, h) if i != "final" and i >= S else None)
            cap.add_document(got)
        return cap.state(S)

    with torch.no_grad():
        state = capture([c1.calibration_ids()])
        state2 = capture(c1.two_documents())
        fit = OR.RidgeFit(state)
        maps = {i: fit.layer(i, (c1.LAM,))[c1.LAM] for i in range(S, L)}
        proj = OK.Projector(S, {i: w for i, (w, _) in maps.items()}, {i: b for i, (_, b) in maps.items()})
        ids = c1.prompt_ids()
        hs, lower = OK.run_lower(m, ids, {S})
        runs = {}
        lg, cache, P = OK.finish(m, ids, hs[S], lower, OK.Arm("kva", split=S, tail=c1.TAIL, fill="proj",
                                                               projector=proj), c1.KEEP)
        runs["proj"] = (lg, cache, P, None)
        lg, cache, P = OK.finish(m, ids, hs[S], lower, OK.Arm("noproj", split=S, tail=c1.TAIL, fill="identity"),
                                 c1.KEEP)
        runs["identity"] = (lg, cache, P, None)
        row_inputs = {}
        lg, cache, P = OK.finish(m, ids, hs[S], lower, OK.Arm("kva", split=S, tail=c1.TAIL, fill="proj",
                                                               projector=proj), c1.KEEP,
                                 exact_rows=c1.exact_rows(), row_inputs=row_inputs)
        runs["exact"] = (lg, cache, P, row_inputs)
    out = c1.summarise(state, state2, maps, runs)
    out["h_split_u"] = (hs[S].double() @ c1.probes(100, m.hidden)).numpy()
    return dict(arrays=out, model=m, state=state, state2=state2, fit=fit, maps=maps, hs=hs, lower=lower, ids=ids,
                proj=proj, calibration=cal_inputs(m))


def cal_inputs(m):
    """The calibration document's split-layer rows and late-layer inputs {layer: [4096, H]} (fp32)."""
    got = {}
    with torch.no_grad():
        m.forward_exact(c1.calibration_ids(),
                        hook=lambda i, h: got.__setitem__(i, h) if i != "final" and i >= c1.SPLIT else None)
    return got


def test_fixture_covers_every_group(gold):
    for key in ("cx", "two_cx", "w_u_5", "proj_k_u_5", "identity_logits_u", "exact_hr_7", "h_split_u"):
        assert key in gold, key
    assert int(gold["proj_P"]) == c1.N_PROMPT - c1.TAIL and int(gold["n"]) == c1.N_CAL


def test_lower_layers_match(gold, run):
    assert rel(run["arrays"]["h_split_u"], gold["h_split_u"]) < RTOL


@pytest.mark.parametrize("tag", ["", "two_"])
def test_capture_sums_match(gold, run, tag):
    a = run["arrays"]
    keys = [k for k in gold if k.startswith(tag) and (tag or not k.startswith(("two_", "proj_", "identity_",
                                                                                 "exact_", "w_", "bias_", "h_")))]
    assert len(keys) > 10
    for k in keys:
        if gold[k].ndim == 0:
            assert int(a[k]) == int(gold[k]), k
        else:
            assert rel(a[k], gold[k]) < 1e-6 or np.abs(a[k] - gold[k]).max() < 1e-9, (k, rel(a[k], gold[k]))


def test_capture_shift_is_the_first_documents_mean(gold, run):
    """Positive control: shifting the two-document capture by the overall mean (a plausible misreading)
    changes the stored shift and first sums, which the fixture resolves."""
    st = run["state2"]
    overall = st["cx"] + st["sx"] / st["n"]
    assert rel(overall.numpy(), gold["two_cx"]) > 1e-3
    assert np.abs(gold["two_sx"]).max() > 1.0           # the first document's mean is not the overall one


def test_ridge_maps_match(gold, run):
    a = run["arrays"]
    for i in range(c1.SPLIT, c1.CONFIG["num_hidden_layers"]):
        for k in (f"w_u_{i}", f"w_tv_{i}", f"w_row0_{i}", f"bias_{i}"):
            assert rel(a[k], gold[k]) < 1e-5, (k, rel(a[k], gold[k]))


def test_ridge_lambda_scale_control(gold, run):
    """Positive control: lambda scaled by the uncentred scatter's mean diagonal gives other maps."""
    st = run["state"]
    fit = OR.RidgeFit(st)
    sxx_unc = st["sxx"].double() + st["n"] * torch.outer(st["cx"].double(), st["cx"].double())
    fit.scale = sxx_unc.diagonal().mean().item()
    w, _ = fit.layer(c1.SPLIT, (c1.LAM,))[c1.LAM]
    got = (w.double() @ c1.probes(100, 256)).numpy()
    assert rel(got, gold[f"w_u_{c1.SPLIT}"]) > 1e-3


@pytest.mark.parametrize("name", ["proj", "identity", "exact"])
def test_finish_matches(gold, run, name):
    a = run["arrays"]
    assert int(a[f"{name}_P"]) == int(gold[f"{name}_P"])
    assert (a[f"{name}_argmax"] == gold[f"{name}_argmax"]).all()
    for k in (f"{name}_logits_u", f"{name}_logits_last"):
        assert rel(a[k], gold[k]) < RTOL, (k, rel(a[k], gold[k]))
    for i in range(c1.SPLIT, c1.CONFIG["num_hidden_layers"]):
        assert int(a[f"{name}_n_{i}"]) == int(gold[f"{name}_n_{i}"]) == c1.N_PROMPT
        for part in ("k", "v"):
            for k in (f"{name}_{part}_u_{i}", f"{name}_{part}_rows_{i}"):
                assert rel(a[k], gold[k]) < RTOL, (k, rel(a[k], gold[k]))
        if name == "exact":
            assert rel(a[f"exact_hr_{i}"], gold[f"exact_hr_{i}"]) < RTOL


def test_exact_rows_change_the_fill(gold):
    """Positive control on the fixture itself: the exact rows' cache slots differ between the plain and
    the exact-row ridgefill arms from the first late layer on (their inputs are scattered in)."""
    rows = c1.exact_rows().numpy()
    i = c1.SPLIT
    diff = np.abs(gold[f"proj_k_u_{i}"] - gold[f"exact_k_u_{i}"]).max(0)       # [n] over heads
    assert (diff[rows] > 1e-4).all()
    others = np.setdiff1d(np.arange(c1.N_PROMPT - c1.TAIL), rows)
    assert diff[others].max() < 1e-6                    # the other prefix rows are the same fill
