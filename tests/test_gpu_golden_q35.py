"""The device's finish() on the Qwen3.5-style hybrid against the reference's own finish() outputs
(tests/golden/finish_q35.npz, written by tests/golden/make_golden.py from the reference in fp32): the
tiny hybrid of tests/golden/q35.py (GDN layers 4..6, gated attention layer 7) in bf16 on the GPU, its
split-layer rows from the oracle's fp32 lower layers (pinned to the same fixture's reads and logits).

Arms (code/kva/kva.py:319-460): fill_by_type {'attention': 'proj', 'gdn': 'identity'} with st corrections
(and its fill_store, taken before + st), the same arm reusing the fill of the arm without st (fill_reuse),
keep_cache=False, the by-type arm with 6 exact rows, and the kvexact arm {'attention': 'oracle',
'gdn': 'proj'} from the true late-layer inputs. Bars as the other hybrid finish tests: 1e-2 relative
Frobenius on logits, K / V and the GDN states right after the fill; 2e-2 on the GDN states after the tail
has run every late layer; argmax agreement above 0.9."""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import q35  # noqa: E402

from oracle import kva as OK  # noqa: E402
from oracle.model import OracleModel  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-2


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(q35.FIXTURE))


@pytest.fixture(scope="module")
def lower():
    """The oracle's fp32 split-layer rows and the true late-layer inputs of the prefix (for kvexact)."""
    om = OracleModel(q35.CONFIG, q35.tensors(), dtype=torch.float32)
    ids = q35.prompt_ids()
    S = q35.SPLIT
    P = ids.shape[0] - q35.TAIL
    store = {}
    with torch.no_grad():
        hs, low = OK.run_lower(om, ids, {S})
        OK.finish(om, ids, hs[S], low, OK.Arm("exact", split=S), q35.KEEP, hook=lambda i, h: store.__setitem__(i, h[:P]))
    return dict(ids=ids, hs=hs[S], store=store)


def _cpu(cache):
    """A cache list (or a fill_store dict {layer: cache}) with its tensors on the host."""
    host = lambda c: {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}   # noqa: E731
    if isinstance(cache, dict):
        return {i: host(c) for i, c in cache.items()}
    return [host(c) for c in cache]


def _arm(name, dev, **kw):
    from rfill.kva import Arm, Projector
    maps = q35.maps()
    proj = Projector(q35.SPLIT, {i: w.to(dev, torch.bfloat16) for i, (w, _) in maps.items()},
                     {i: b.to(dev, torch.bfloat16) for i, (_, b) in maps.items()})
    base = dict(split=q35.SPLIT, tail=q35.TAIL, fill="by_type", projector=proj,
                fill_by_type={"attention": "proj", "gdn": "identity"})
    base.update(kw)
    return Arm(name, **base)


def _check(gold, name, lg, cache, P, types, state_tol):
    u_v = q35.probes(105, q35.VOCAB, 4)
    lg = lg.double().cpu()
    el = rel((lg @ u_v).numpy(), gold[f"{name}_logits_u"])
    agree = float((lg.argmax(-1).numpy() == gold[f"{name}_argmax"]).mean())
    mine = q35.cache_arrays(name, _cpu(cache), P, types)
    errs = {}
    for k, v in mine.items():
        assert k in gold, k
        if v.ndim == 0:
            assert int(v) == int(gold[k]), k
        else:
            errs[k] = rel(v, gold[k])
    print(f"{name}: logits {el:.2e}, argmax agreement {agree:.3f}, worst cache "
          f"{max(errs.values()) if errs else 0.0:.2e}")
    assert el < TOL and agree > 0.9
    for k, e in errs.items():
        assert e < (state_tol if "_rec_" in k else TOL), (k, e)


@pytest.mark.parametrize("name", ["st", "reuse", "nokeep", "exact", "kvexact"])
def test_hybrid_finish_matches_reference(dev, gold, lower, name):
    from rfill.kva import finish
    from rfill.model import FillModel
    S = q35.SPLIT
    model = FillModel(q35.CONFIG, q35.tensors(), dev, layers=list(range(S, q35.L)))
    ids, hs = lower["ids"], lower["hs"]
    st = {i: t.to(dev) for i, t in q35.st().items()}
    kw, arm = {}, None
    if name == "st":
        store = {}
        arm, kw = _arm("kva+st", dev, st=st), dict(fill_store=store)
    elif name == "reuse":
        base = {}
        finish(model, ids, hs, None, _arm("kva", dev), q35.KEEP, fill_store=base)
        arm, kw = _arm("kva+st", dev, st=st), dict(fill_reuse=base)
    elif name == "nokeep":
        arm, kw = _arm("kva+st", dev, st=st), dict(keep_cache=False)
    elif name == "exact":
        arm, kw = _arm("kva", dev), dict(exact_rows=q35.exact_rows())
    else:
        arm = _arm("kvexact", dev, fill_by_type={"attention": "oracle", "gdn": "proj"})
        kw = dict(oracle={i: t.to(dev, torch.bfloat16) for i, t in lower["store"].items()})
    lg, cache, P = finish(model, ids, hs, None, arm, q35.KEEP, **kw)
    torch.cuda.synchronize()
    assert P == int(gold[f"{name}_P"])
    types = model.layer_types
    _check(gold, name, lg, cache, P, types, 2e-2)
    if name == "st":                  # the fill_store snapshot: right after the fill, before + st
        mine = q35.cache_arrays("st_store", _cpu(store), P, types)
        for k, v in mine.items():
            if v.ndim:
                assert rel(v, gold[k]) < TOL, (k, rel(v, gold[k]))
    if name == "nokeep":
        assert all(cache[i] == {} for i in range(S, q35.L))
