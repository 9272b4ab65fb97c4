"""Oracle of the fit driver (test infrastructure; see oracle/__init__.py).

Restates code/scripts/fit_sweep.py: the capture pass over calibration documents (:236-248) with
capture_hook's sums (:87-144, via oracle.ridge.Capture), the fit of every late layer for each lambda of
LAMBDAS (:44, :286-293; maps rounded to bf16 as :292), and the held-out lambda selection by read cosine
(:298-318): for each held-out document and late layer i, the reads (pre-RoPE K / V, k-normed where the
model norms K) of the true layer input h_i against the reads of each candidate's prediction from h_S
(F.linear with the bf16 map, or h_S itself for "identity"); per document the mean cosine over rows and KV
heads, averaged over K and V; per candidate and layer the mean over documents; the chosen lambda
maximises the mean over layers, the first such in LAMBDAS order (Python's max)."""
import torch
import torch.nn.functional as F

from . import ridge

LAMBDAS = (1e-4, 3e-4, 1e-3, 3e-3, 0.01, 0.03, 0.1, 0.3, 1.0)      # fit_sweep.py:44


def _inputs(model, ids, first):
    """{layer: input h} of every layer >= first over one document's exact forward."""
    got = {}
    model.forward_exact(ids, hook=lambda i, h: got.__setitem__(i, h) if i != "final" and i >= first else None)
    return got


def capture(model, docs, splits):
    """oracle.ridge.Capture over the documents' exact forwards (fit_sweep.py:236-248)."""
    cap = ridge.Capture(splits, model.n_layers, model.hidden)
    for ids in docs:
        cap.add_document(_inputs(model, ids, min(splits)))
    return cap


def fit_maps(state, lambdas=LAMBDAS):
    """{lam: {layer: (W [d_out, d_in] bf16, b [d_out] bf16)}} (fit_sweep.py:286-293)."""
    fit = ridge.RidgeFit(state)
    maps = {lam: {} for lam in lambdas}
    for i in state["layers"]:
        for lam, (w, b) in fit.layer(i, lambdas).items():
            maps[lam][i] = (w.to(torch.bfloat16), b.to(torch.bfloat16))
    return maps


def read_scores(model, held, split, maps):
    """{candidate: {layer: mean read cosine}} over the held-out documents (fit_sweep.py:298-314);
    candidates: the lambdas of maps, then "identity"."""
    late = list(range(split, model.n_layers))
    cand = list(maps) + ["identity"]
    sums = {c: {i: 0.0 for i in late} for c in cand}
    for ids in held:
        got = _inputs(model, ids, split)
        hs = got[split]
        for i in late:
            true = model.reads(i, got[i])
            for c in cand:
                if c == "identity":
                    x = hs
                else:
                    w, b = maps[c][i]
                    x = F.linear(hs, w.to(hs.dtype), b.to(hs.dtype))
                pred = model.reads(i, x)
                sums[c][i] += sum(F.cosine_similarity(pred[r].float(), true[r].float(), dim=-1).mean().item()
                                  for r in true) / len(true)
    return {c: {i: v / len(held) for i, v in s.items()} for c, s in sums.items()}


def best_lambda(scores, lambdas=LAMBDAS):
    """The lambda with the highest mean over layers, the first in lambdas order on ties (fit_sweep.py:315-318)."""
    mean = {c: sum(v.values()) / len(v) for c, v in scores.items()}
    return max(lambdas, key=lambda lam: mean[lam])
