"""Pins the oracle of the fit driver (oracle/fit.py, code/scripts/fit_sweep.py:236-318) on the CPU:
documents weigh equally in the read-cosine score whatever their length, the identity candidate scores 1
at the split layer, the reads are the cached keys before RoPE, and ties go to the first lambda."""
import math

import torch

from fill_cases import case
from oracle import fit as OF
from oracle import model as OM
from oracle import ops as OO


class _Stub:
    """A two-layer 'model' whose layer inputs are given per document: h_0 = e_0 rows, h_1 = rows at angle
    theta_doc from e_0; reads(i, x) = x itself as one K and one V head of width 2."""
    n_layers = 2

    def __init__(self, angles):
        self.angles = angles

    def forward_exact(self, ids, hook=None):
        n = ids.numel()
        th = self.angles[int(ids[0])]
        h0 = torch.zeros(n, 2)
        h0[:, 0] = 1.0
        h1 = torch.tensor([[math.cos(th), math.sin(th)]]).repeat(n, 1)
        hook(0, h0)
        hook(1, h1)
        hook("final", h1)
        return None, None

    def reads(self, i, x):
        return dict(k=x.view(-1, 1, 2), v=x.view(-1, 1, 2))


def test_documents_weigh_equally():
    """Doc 0 (1 row) at angle 0 scores cos 0 = 1, doc 1 (3 rows) at 90 degrees scores 0: the mean over
    documents is 0.5 (a pooled mean over rows would give 0.25). A map that rotates e_0 onto e_1 scores
    the reverse: 0 and 1, mean 0.5 again; one that maps e_0 to -e_0 scores -1 on doc 0."""
    model = _Stub({0: 0.0, 1: math.pi / 2})
    held = [torch.tensor([0]), torch.tensor([1, 1, 1])]
    rot = (torch.tensor([[0.0, 0.0], [1.0, 0.0]]), torch.zeros(2))          # x W^T: e_0 -> e_1
    neg = (-torch.eye(2), torch.zeros(2))
    s = OF.read_scores(model, held, 0, {0.1: {0: rot, 1: rot}, 0.2: {0: neg, 1: neg}})
    assert abs(s["identity"][1] - 0.5) < 1e-6
    assert abs(s[0.1][1] - 0.5) < 1e-6
    assert abs(s[0.2][1] - (-1.0 + 0.0) / 2) < 1e-6
    assert abs(s["identity"][0] - 1.0) < 1e-6 and abs(s[0.2][0] + 1.0) < 1e-6


def test_identity_scores_one_at_the_split():
    cfg, t = case("llama_c1", layers=3)
    om = OM.OracleModel(cfg, t, dtype=torch.float32)
    g = torch.Generator().manual_seed(5)
    held = [torch.randint(0, 64, (n,), generator=g) for n in (40, 25)]
    maps = {1e-2: {i: (torch.eye(256) * 0.5, torch.zeros(256)) for i in (1, 2)}}
    s = OF.read_scores(om, held, 1, maps)
    assert abs(s["identity"][1] - 1.0) < 1e-6
    # a map that halves every row leaves every cosine unchanged up to the norm: the score is 1 too
    assert abs(s[1e-2][1] - 1.0) < 1e-5
    assert s["identity"][2] < 1.0 - 1e-4


def test_reads_are_the_cached_keys_before_rope():
    """reads(i, h) K with RoPE applied, and V, equal the K / V the layer appends to its cache (pinned
    against transformers' models); for Qwen3 the K head norm is inside."""
    for name in ("llama_c1", "qwen3_knorm"):
        cfg, t = case(name)
        om = OM.OracleModel(cfg, t, dtype=torch.float32)
        g = torch.Generator().manual_seed(6)
        h = torch.randn(33, cfg["hidden_size"], generator=g)
        pos = torch.arange(33)
        c = om.new_cache()
        om.fill(0, h, pos, c)
        r = om.reads(0, h)
        cos, sin = OO.rope_cos_sin(om.inv_freq, pos, h.dtype)
        k = OO.apply_rope(r["k"].transpose(0, 1), cos, sin)
        torch.testing.assert_close(k, c[0]["k"], rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(r["v"].transpose(0, 1), c[0]["v"], rtol=0, atol=0)


def test_best_lambda_takes_the_first_maximum():
    s = {1e-3: {5: 0.9, 6: 0.8}, 1e-2: {5: 0.8, 6: 0.9}, 0.1: {5: 0.7, 6: 0.7}, "identity": {5: 1.0, 6: 1.0}}
    assert OF.best_lambda(s, (1e-3, 1e-2, 0.1)) == 1e-3
    assert OF.best_lambda(s, (0.1, 1e-2, 1e-3)) == 1e-2
    assert OF.best_lambda(s, (0.1,)) == 0.1


def test_capture_is_the_capture_sums_over_forward_inputs():
    """oracle.fit.capture == oracle.ridge.Capture fed every layer input >= the smallest split."""
    cfg, t = case("llama_c1", layers=3)
    om = OM.OracleModel(cfg, t, dtype=torch.float32)
    g = torch.Generator().manual_seed(7)
    docs = [torch.randint(0, 64, (n,), generator=g) for n in (30, 12)]
    cap = OF.capture(om, docs, [2, 1])
    want = OF.ridge.Capture([1, 2], 3, 256)
    for ids in docs:
        got = {}
        om.forward_exact(ids, hook=lambda i, h: got.__setitem__(i, h) if i != "final" else None)
        want.add_document({i: h for i, h in got.items() if i >= 1})
    for S in (1, 2):
        a, b = cap.state(S), want.state(S)
        assert a["layers"] == b["layers"] == list(range(S, 3)) and a["n"] == b["n"] == 42
        torch.testing.assert_close(a["sxx"], b["sxx"], rtol=0, atol=0)
        for i in a["layers"]:
            torch.testing.assert_close(a["sxy"][i], b["sxy"][i], rtol=0, atol=0)
