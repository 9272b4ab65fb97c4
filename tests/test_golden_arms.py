"""The oracle's finish() branches and Qwen3.5 reads against golden vectors the reference wrote itself
(tests/golden/make_golden.py), in fp32 on the CPU, plus the invariants the reference's own tests hold.

tests/golden/finish_c1_arms.npz (the tiny Llama-style workload of tests/golden/c1.py):
  * fill 'none' with 18 exact rows: only the rows reach the late layers (code/kva/kva.py:406-411);
  * fill 'oracle' from the true late-layer inputs oracle_tap keeps in the exact arm (code/kva/kva.py:310-316,
    :418-419).
tests/golden/finish_q35.npz (the tiny Qwen3.5-style hybrid of tests/golden/q35.py):
  * Qwen35.reads of GDN layers (pre-conv q / k / v, [b | a]) and of the gated attention layer, and the
    held-out read cosine per layer (code/kva/model.py:558-571, code/scripts/fit_sweep.py:307-313);
  * finish() with fill_by_type {'attention': 'proj', 'gdn': 'identity'} and st, fill_store, fill_reuse,
    keep_cache=False, exact rows through GDN layers, and the kvexact arm {'attention': 'oracle', 'gdn': 'proj'}.
Invariants (code/tests/test_qwen3.py:117-128, :167-168; code/tests/test_multiturn.py:171-196): the tail
covering the whole prompt is the exact forward bit for bit; the 'oracle' fill writes the exact forward's
prefix caches; every prefix row exact gives the exact caches.
Each group has a positive control: a plausible mistake planted in the oracle's inputs fails the same check."""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import c1  # noqa: E402
import q35  # noqa: E402

from oracle import kva as OK  # noqa: E402
from oracle import ops as oops  # noqa: E402
from oracle.model import OracleModel  # noqa: E402

RTOL = 1e-4


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


# ------------------------------------------------------------------ C1: fill 'none' and fill 'oracle'

@pytest.fixture(scope="module")
def c1_gold():
    return dict(np.load(c1.FIXTURE.with_name("finish_c1_arms.npz")))


@pytest.fixture(scope="module")
def c1_run():
    m = OracleModel(c1.CONFIG, c1.tensors(), dtype=torch.float32)
    S = c1.SPLIT
    ids = c1.prompt_ids()
    with torch.no_grad():
        hs, lower = OK.run_lower(m, ids, {S})
        P = ids.shape[0] - c1.TAIL
        store = {}

        def tap(i, h):
            store[i] = h[:P]
        exact = OK.finish(m, ids, hs[S], lower, OK.Arm("exact", split=S), c1.KEEP, hook=tap)
    return dict(m=m, ids=ids, hs=hs, lower=lower, store=store, exact=exact, P=P)


def _u(t, seed, width):
    return (t.double() @ c1.probes(seed, width)).numpy()


def test_fill_none_with_exact_rows_matches(c1_gold, c1_run):
    m, S = c1_run["m"], c1.SPLIT
    row_inputs = {}
    with torch.no_grad():
        lg, cache, P = OK.finish(m, c1_run["ids"], c1_run["hs"][S], c1_run["lower"],
                                 OK.Arm("none", split=S, tail=c1.TAIL, fill="none"), c1.KEEP,
                                 exact_rows=c1.exact_rows(), row_inputs=row_inputs)
    g = c1_gold
    assert P == int(g["none_P"]) and (lg.argmax(-1).numpy() == g["none_argmax"]).all()
    assert rel((lg.double() @ c1.probes(103, 1024, 4)).numpy(), g["none_logits_u"]) < RTOL
    for i in range(S, m.n_layers):
        assert cache[i]["n"] == int(g[f"none_n_{i}"]) == c1.N_EXACT + c1.TAIL
        for part in ("k", "v"):
            assert rel(_u(cache[i][part], 102, 64), g[f"none_{part}_u_{i}"]) < RTOL, (i, part)
        assert rel(_u(row_inputs[i], 100, m.hidden), g[f"none_hr_u_{i}"]) < RTOL


def test_fill_none_control_rows_at_their_positions(c1_gold, c1_run):
    """Positive control: the exact rows run the first late layer at positions 0 .. R - 1 (their index
    among the rows, a plausible slip) instead of their prompt positions: the keys differ."""
    m, S = c1_run["m"], c1.SPLIT
    rows = c1.exact_rows()
    cache = [dict(c) for c in c1_run["lower"][:S]] + [dict() for _ in range(m.n_layers - S)]
    with torch.no_grad():
        m.layer(S, c1_run["hs"][S][rows], torch.arange(rows.numel()), cache)
    got = _u(cache[S]["k"], 102, 64)
    want = c1_gold[f"none_k_u_{S}"][:, :rows.numel()]
    assert rel(got, want) > 1e-2


def test_fill_oracle_matches(c1_gold, c1_run):
    m, S, store = c1_run["m"], c1.SPLIT, c1_run["store"]
    g = c1_gold
    assert rel((c1_run["exact"][0].double() @ c1.probes(103, 1024, 4)).numpy(), g["exact_logits_u"]) < RTOL
    with torch.no_grad():
        lg, cache, P = OK.finish(m, c1_run["ids"], c1_run["hs"][S], c1_run["lower"],
                                 OK.Arm("oracle", split=S, tail=c1.TAIL, fill="oracle"), c1.KEEP, oracle=store)
    assert P == int(g["oracle_P"]) and (lg.argmax(-1).numpy() == g["oracle_argmax"]).all()
    assert rel((lg.double() @ c1.probes(103, 1024, 4)).numpy(), g["oracle_logits_u"]) < RTOL
    for i in range(S, m.n_layers):
        assert rel(_u(store[i], 100, m.hidden), g[f"oracle_in_u_{i}"]) < RTOL
        for part in ("k", "v"):
            assert rel(_u(cache[i][part], 102, 64), g[f"oracle_{part}_u_{i}"]) < RTOL
    # the reference's own outputs hold the invariant: the 'oracle' fill writes the exact prefill
    for i in range(S, m.n_layers):
        for part in ("k", "v"):
            assert rel(g[f"oracle_{part}_u_{i}"], g[f"exact_{part}_u_{i}"]) < 1e-5


def test_fill_oracle_control_next_layers_inputs(c1_gold, c1_run):
    """Positive control: filling layer i from the inputs of layer i + 1 (an off-by-one in the tap) fails."""
    m, S, store = c1_run["m"], c1.SPLIT, c1_run["store"]
    shifted = {i: store.get(i + 1, store[i]) for i in store}
    with torch.no_grad():
        _, cache, _ = OK.finish(m, c1_run["ids"], c1_run["hs"][S], c1_run["lower"],
                                OK.Arm("oracle", split=S, tail=c1.TAIL, fill="oracle"), c1.KEEP, oracle=shifted)
    assert rel(_u(cache[S]["k"], 102, 64), c1_gold[f"oracle_k_u_{S}"]) > 1e-2


def test_invariant_tail_over_the_whole_prompt_is_the_exact_forward(c1_run):
    """code/tests/test_qwen3.py:167-168: tail = N gives P = 0 and the exact forward's logits bit for bit."""
    m, S, ids = c1_run["m"], c1.SPLIT, c1_run["ids"]
    n = ids.shape[0]
    with torch.no_grad():
        full, _, P = OK.finish(m, ids, c1_run["hs"][S], c1_run["lower"],
                               OK.Arm("kva", split=S, tail=n, fill="identity"), c1.KEEP)
        exact, _ = m.forward_exact(ids, keep=torch.arange(n - c1.KEEP, n))
    assert P == 0 and torch.equal(full, exact)


def test_invariant_oracle_fill_and_all_rows_exact_give_the_exact_caches(c1_run):
    """code/tests/test_qwen3.py:117-128 (fill writes the exact layer's cache) and code/tests/test_multiturn.py:
    191-196 (every prefix row exact gives the exact cache): both against the exact arm's caches."""
    m, S, ids, P = c1_run["m"], c1.SPLIT, c1_run["ids"], c1_run["P"]
    ecache = c1_run["exact"][1]
    with torch.no_grad():
        _, ocache, _ = OK.finish(m, ids, c1_run["hs"][S], c1_run["lower"],
                                 OK.Arm("oracle", split=S, tail=c1.TAIL, fill="oracle"), c1.KEEP,
                                 oracle=c1_run["store"])
        _, rcache, _ = OK.finish(m, ids, c1_run["hs"][S], c1_run["lower"],
                                 OK.Arm("noproj", split=S, tail=c1.TAIL, fill="identity"), c1.KEEP,
                                 exact_rows=torch.arange(P))
    for i in range(S, m.n_layers):
        for part in ("k", "v"):
            want = ecache[i][part]
            torch.testing.assert_close(ocache[i][part], want, atol=1e-5, rtol=1e-5)
            torch.testing.assert_close(rcache[i][part], want, atol=1e-5, rtol=1e-5)


# ------------------------------------------------------------------ the hybrid: reads and finish arms

@pytest.fixture(scope="module")
def q_gold():
    return dict(np.load(q35.FIXTURE))


@pytest.fixture(scope="module")
def q_model():
    return OracleModel(q35.CONFIG, q35.tensors(), dtype=torch.float32)


@pytest.fixture(scope="module")
def q_reads(q_model):
    m, S = q_model, q35.SPLIT
    got = {}
    with torch.no_grad():
        m.forward_exact(q35.held_ids(), hook=lambda i, h: got.__setitem__(i, h) if i != "final" and i >= S else None)
    return got


def test_reads_match_the_reference(q_gold, q_model, q_reads):
    m, S, got = q_model, q35.SPLIT, q_reads
    maps = q35.maps()
    with torch.no_grad():
        for i in range(S, m.n_layers):
            true = m.reads(i, got[i])
            pred = m.reads(i, torch.nn.functional.linear(got[S], maps[i][0], maps[i][1]))
            ident = m.reads(i, got[S])
            assert sorted(true) == (["k", "v"] if m.layer_types[i] == "attn" else ["ba", "k", "q", "v"])
            for tag, r in (("true", true), ("pred", pred)):
                mine = q35.read_arrays(f"{tag}_{i}", r)
                for k, v in mine.items():
                    assert rel(v, q_gold[k]) < 1e-5, (k, rel(v, q_gold[k]))
            assert abs(q35.cosine_score(pred, true) - float(q_gold[f"score_proj_{i}"])) < 1e-6
            assert abs(q35.cosine_score(ident, true) - float(q_gold[f"score_identity_{i}"])) < 1e-6
    assert float(q_gold[f"score_identity_{S}"]) > 0.999999          # h_S is layer S's own input


def test_reads_control_post_conv(q_gold, q_model, q_reads):
    """Positive control: GDN reads taken after the causal conv (a plausible misreading of 'the inputs that
    feed the state') differ from the reference's pre-conv reads."""
    m, i = q_model, q35.SPLIT
    w = m.W[i]
    with torch.no_grad():
        pre, _, _ = m.gdn_inputs(i, m.in_norm(q_reads[i], w["ln1"]))
        y, _ = oops.causal_conv(pre, None, w["conv"])
    kd = q35.NK * q35.DK
    q = y[:, :kd].reshape(-1, q35.NK, q35.DK)
    got = q35.read_arrays("x", {"q": q})["x_q_u"]
    assert rel(got, q_gold[f"true_{i}_q_u"]) > 1e-2


def _arm(name, **kw):
    proj = q35.maps()
    P = OK.Projector(q35.SPLIT, {i: w for i, (w, _) in proj.items()}, {i: b for i, (_, b) in proj.items()})
    base = dict(split=q35.SPLIT, tail=q35.TAIL, fill="by_type", projector=P,
                fill_by_type={"attention": "proj", "gdn": "identity"})
    base.update(kw)
    return OK.Arm(name, **base)


@pytest.fixture(scope="module")
def q_runs(q_model):
    m, S = q_model, q35.SPLIT
    ids = q35.prompt_ids()
    st = q35.st()
    runs, stores = {}, {}
    with torch.no_grad():
        hs, lower = OK.run_lower(m, ids, {S})
        stores["st"], sb = {}, {}
        runs["st"] = OK.finish(m, ids, hs[S], lower, _arm("kva+st", st=st), q35.KEEP, fill_store=stores["st"])
        runs["base"] = OK.finish(m, ids, hs[S], lower, _arm("kva"), q35.KEEP, fill_store=sb)
        runs["reuse"] = OK.finish(m, ids, hs[S], lower, _arm("kva+st", st=st), q35.KEEP, fill_reuse=sb)
        runs["nokeep"] = OK.finish(m, ids, hs[S], lower, _arm("kva+st", st=st), q35.KEEP, keep_cache=False)
        row_inputs = {}
        runs["exact"] = OK.finish(m, ids, hs[S], lower, _arm("kva"), q35.KEEP, exact_rows=q35.exact_rows(),
                                  row_inputs=row_inputs)
        P = ids.shape[0] - q35.TAIL
        store = {}
        OK.finish(m, ids, hs[S], lower, OK.Arm("exact", split=S), q35.KEEP,
                  hook=lambda i, h: store.__setitem__(i, h[:P]))
        runs["kvexact"] = OK.finish(m, ids, hs[S], lower,
                                    _arm("kvexact", fill_by_type={"attention": "oracle", "gdn": "proj"}), q35.KEEP,
                                    oracle=store)
    return dict(runs=runs, stores=stores, row_inputs=row_inputs, m=m)


def _check_run(gold, name, lg, cache, P, types, tol=RTOL):
    assert P == int(gold[f"{name}_P"])
    assert (lg.argmax(-1).numpy() == gold[f"{name}_argmax"]).all()
    u_v = q35.probes(105, q35.VOCAB, 4)
    assert rel((lg.double() @ u_v).numpy(), gold[f"{name}_logits_u"]) < tol
    assert rel(lg[-1].double().numpy(), gold[f"{name}_logits_last"]) < tol
    mine = q35.cache_arrays(name, cache, P, types)
    assert len(mine) >= q35.L - q35.SPLIT and all(k in gold for k in mine), name
    for k, v in mine.items():
        if v.ndim == 0:
            assert int(v) == int(gold[k]), k
        else:
            assert rel(v, gold[k]) < tol, (k, rel(v, gold[k]))


@pytest.mark.parametrize("name", ["st", "base", "reuse", "nokeep", "exact", "kvexact"])
def test_hybrid_finish_arms_match(q_gold, q_runs, name):
    lg, cache, P = q_runs["runs"][name]
    _check_run(q_gold, name, lg, cache, P, q_runs["m"].layer_types)
    if name == "exact":
        u_h = q35.probes(100, q35.H)
        for i in range(q35.SPLIT, q35.L):
            assert rel((q_runs["row_inputs"][i].double() @ u_h).numpy(), q_gold[f"exact_hr_u_{i}"]) < RTOL
    if name == "nokeep":
        assert all(int(q_gold[f"nokeep_dropped_{i}"]) == 1 for i in range(q35.SPLIT, q35.L))


def test_hybrid_fill_store_is_taken_before_st(q_gold, q_runs):
    """fill_store keeps each late layer's cache right after the fill, before + st: the oracle's store matches
    the reference's, and its GDN states differ from the states with st added (positive control)."""
    types = q_runs["m"].layer_types
    store = q_runs["stores"]["st"]
    P = q_runs["runs"]["st"][2]
    mine = q35.cache_arrays("st_store", store, P, types)
    for k, v in mine.items():
        if v.ndim:
            assert rel(v, q_gold[k]) < RTOL, k
    st = q35.st()
    i = q35.SPLIT
    plus = q35.cache_arrays("x", {j: (dict(store[j], rec=store[j]["rec"] + st[j]) if j in st else store[j])
                                  for j in range(q35.SPLIT, q35.L)}, P, types)
    assert rel(plus[f"x_rec_u_{i}"], q_gold[f"st_store_rec_u_{i}"]) > 1e-3


def test_hybrid_reuse_and_nokeep_give_the_st_arms_logits(q_gold):
    """On the reference's own outputs: reusing the base arm's fill gives the st arm's logits, and dropping the
    caches changes no logit."""
    for name in ("reuse", "nokeep"):
        assert np.array_equal(q_gold[f"{name}_logits_u"], q_gold["st_logits_u"]), name
