"""Oracle of the qattn exact-row selector (test infrastructure; see oracle/__init__.py).

Restates code/kva/select.py: qattn_layers (:217-220), window_mass (:223-245) and top_rows (:311-315),
over the oracle model (its in_norm and queries)."""
import torch

LAYERS = (3, 7, 11, 15)          # select.py:80


def qattn_layers(model, split, layers=None):
    layers = LAYERS if layers is None else layers
    return [L for L in layers if L < split and model.layer_types[L] == "attn"]


@torch.no_grad()
def window_mass(model, win, cache, layers, end=None):
    """Aw mass [n] fp64 (CPU): for each layer L, the window rows win[L] (the w layer-L inputs of rows
    [end - w, end)) as queries over the cached post-RoPE keys of all n rows, dense causal softmax, summed
    over window rows and query heads; fp32 per K / V head group, fp64 over groups and layers."""
    mass = None
    for L in layers:
        k = cache[L]["k"]
        hkv, n, d = k.shape
        h = win[L]
        w = h.shape[0]
        e = n if end is None else end
        qpos = torch.arange(e - w, e)
        q = model.queries(L, model.in_norm(h, model.W[L]["ln1"]), qpos)
        q = q[0] if isinstance(q, tuple) else q
        rep = q.shape[0] // hkv
        mask = torch.arange(n)[None, :] > qpos[:, None]
        acc = torch.zeros(n, dtype=torch.float64)
        for g in range(hkv):
            s = torch.matmul(q[g * rep:(g + 1) * rep].float(), k[g].float().T).mul_(model.scale)
            s.masked_fill_(mask, float("-inf"))
            acc += torch.softmax(s, -1).sum((0, 1)).double()
        mass = acc if mass is None else mass + acc
    return mass


def top_rows(score, P, b):
    """The b highest-scoring rows in [0, P), ties broken by position; sorted."""
    b = max(0, min(int(b), P))
    order = torch.sort(-score[:P].double(), stable=True).indices
    return sorted(order[:b].tolist())
