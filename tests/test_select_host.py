"""The qattn selector's oracle (code/kva/select.py:217-245, 311-315) pinned on the CPU: a float64
brute force over every (layer, head, window row, key) on a small case, the invariants of a dense causal
softmax (each window row and head puts total mass 1 on keys at or before its position; keys at or after
the window's end get none), a positive control (no causal mask changes the mass), and top_rows' ties."""
import math

import torch

from fill_cases import case, inputs
from oracle import model as OM
from oracle import select as OS


def build(n=40, w=8, layers=(1, 3), seed=0):
    cfg, t = case("llama_c1", layers=4, seed=seed)
    om = OM.OracleModel(cfg, t, dtype=torch.float32)
    pos = torch.arange(n)
    xs = {L: inputs(n, cfg["hidden_size"], seed=50 + L).float() for L in layers}
    cache = om.new_cache()
    for L in layers:
        om.fill(L, xs[L], pos, cache)
    return om, cache, xs


def brute(om, cache, xs, layers, w, end):
    mass = [0.0] * cache[layers[0]]["k"].shape[1]
    for L in layers:
        q = om.queries(L, om.in_norm(xs[L][end - w:end], om.W[L]["ln1"]), torch.arange(end - w, end))
        q = (q[0] if isinstance(q, tuple) else q).double()
        k = cache[L]["k"].double()
        hq, hkv = q.shape[0], k.shape[0]
        for h in range(hq):
            kg = k[h // (hq // hkv)]
            for i in range(w):
                p = end - w + i
                s = [float(q[h, i] @ kg[j]) * om.scale for j in range(p + 1)]
                mx = max(s)
                z = sum(math.exp(v - mx) for v in s)
                for j in range(p + 1):
                    mass[j] += math.exp(s[j] - mx) / z
    return torch.tensor(mass, dtype=torch.float64)


def test_window_mass_matches_brute_force():
    om, cache, xs = build()
    layers, w, end = [1, 3], 8, 33
    win = {L: xs[L][end - w:end] for L in layers}
    got = OS.window_mass(om, win, cache, layers, end)
    want = brute(om, cache, xs, layers, w, end)
    assert float((got - want).abs().max() / want.abs().max()) < 1e-5


def test_window_mass_invariants():
    om, cache, xs = build(n=64, w=16)
    layers, w, end = [1, 3], 16, 50
    got = OS.window_mass(om, {L: xs[L][end - w:end] for L in layers}, cache, layers, end)
    assert abs(float(got.sum()) - len(layers) * w * om.n_heads) < 1e-4 * len(layers) * w * om.n_heads
    assert bool((got[end:] == 0).all()) and bool((got[:end] > 0).all())
    # positive control: without the causal mask the window rows also put mass on later keys
    q = om.queries(3, om.in_norm(xs[3][end - w:end], om.W[3]["ln1"]), torch.arange(end - w, end))
    q = q[0] if isinstance(q, tuple) else q
    s = torch.matmul(q[0].float(), cache[3]["k"][0].float().T) * om.scale
    assert float(torch.softmax(s, -1)[:, end:].sum()) > 1e-3


def test_top_rows_ties_by_position():
    s = torch.tensor([1.0, 3.0, 2.0, 3.0, 0.5, 3.0])
    assert OS.top_rows(s, 6, 2) == [1, 3]
    assert OS.top_rows(s, 4, 3) == [1, 2, 3]
    assert OS.top_rows(s, 6, 10) == [0, 1, 2, 3, 4, 5]
    from rfill.select import top_rows
    assert top_rows(s, 6, 2) == [1, 3] and top_rows(s, 5, 4) == [0, 1, 2, 3]


def test_qattn_layers():
    cfg, t = case("llama_c1", layers=16)
    om = OM.OracleModel(cfg, t, dtype=torch.float32)
    assert OS.qattn_layers(om, 10) == [3, 7] and OS.qattn_layers(om, 16) == [3, 7, 11, 15]
    assert OS.qattn_layers(om, 10, layers=(1, 2)) == [1, 2]
