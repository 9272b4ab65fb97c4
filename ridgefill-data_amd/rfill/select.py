"""Exact-row selection by window attention mass, the reference's qattn selector (code/kva/select.py:
217-245, 311-315), with the mass on rf_window_mass.

An arm with meta["select"] = {"kind": "qattn", "budget": b} runs exactly the top round(b * N) prefix rows by
the attention probability the last WINDOW prompt rows give them at the exact lower attention layers
LAYERS below the split (dense causal softmax over every key, summed over the window's query rows and all
query heads). The rows go to finish(exact_rows=...) / fill_late, which scatters them bit-exactly.
"""
import torch

from . import ops
from ._lib import UnsupportedArchitecture

WINDOW = 64                      # code/kva/select.py:79
LAYERS = (3, 7, 11, 15)          # code/kva/select.py:80


def qattn_layers(model, split, layers=None):
    """The exact lower attention layers the selector reads (code/kva/select.py:217-220)."""
    layers = LAYERS if layers is None else layers
    return [L for L in layers if L < split and model.layer_types[L] == "attn"]


@torch.no_grad()
def window_mass(model, win, cache, layers, end=None, workspace=None):
    """Aw attention mass [n] (fp64, CPU) of every row of an n-row prompt (code/kva/select.py:223-245).
    model: a FillModel holding the layers; win {L: the layer-L inputs [w, H] bf16 of the window rows
    [end - w, end)}; cache: the exact lower cache ({L: dict with the post-RoPE keys kbuf [hkv, cap, d] and
    n}); end = n by default. Rows at or after end get no mass. Each layer's queries are rf_norm_q's
    (input norm, q projection, q_norm, RoPE at the window positions); the mass is rf_window_mass's."""
    mass = None
    for L in layers:
        if model.layer_types[L] != "attn":
            raise UnsupportedArchitecture(f"window mass of layer {L}: not an attention layer")
        c = cache[L]
        n = c["n"]
        h = win[L]
        w = h.shape[0]
        e = n if end is None else end
        if not 0 < w <= e <= n:
            raise ValueError(f"window_mass: {w} window rows ending at {e} of {n} cached rows")
        if mass is None:
            mass = torch.zeros(n, dtype=torch.float64, device=h.device)
        wts = model._pack_rows(L)
        qpos = torch.arange(e - w, e, device=h.device)
        ssq = ops.row_ssq(h)
        cs = model.rope_table(qpos)
        q = ops.norm_q(h, ssq, model.eps, wts["wq"], model.n_heads, model.head_dim, wts.get("q_norm"),
                       model.knorm_kind, cs, torch.arange(w, device=h.device),
                       workspace=model.gemm_workspace(w, wts["wq"].shape[0], h.shape[1], h.device))
        ops.window_mass(q, e - w, c["kbuf"], model.n_heads, model.scale, mass, workspace=workspace)
    return mass.cpu()


def top_rows(score, P, b):
    """The b highest-scoring rows in [0, P), ties broken by position; sorted (code/kva/select.py:311-315)."""
    b = max(0, min(int(b), P))
    order = torch.sort(-score[:P].double(), stable=True).indices
    return sorted(order[:b].tolist())


def qattn_rows(model, win, cache, split, P, n, budget=0.05, layers=None, end=None):
    """The qattn selector's rows for one prompt: top round(budget * n) of [0, P) by window_mass at
    qattn_layers(model, split, layers) (code/kva/select.py:365-366, 394-397)."""
    mass = window_mass(model, win, cache, qattn_layers(model, split, layers), end)
    return top_rows(mass, P, round(budget * n))
