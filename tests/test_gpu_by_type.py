"""GPU parity of finish()'s per-layer-type fills and fill reuse (code/kva/kva.py:108-115, :319-460) against the
oracle's finish:
  * a llama.cpp adapter (GGUF: an F16 map for the late attention layer, native GDN layers with F32 st
    corrections) loaded by load_gguf drives a hybrid's finish() through adapter_arm: fill_by_type
    {'attention': 'proj', 'gdn': 'identity'} plus st, with and without exact rows;
  * the hybrid arm of the reference's kvexact kind, {'attention': 'oracle', 'gdn': 'proj'}, from given true inputs;
  * fill 'none' with exact rows (only the rows reach the late layers);
  * fill_store / fill_reuse: an arm reusing a stored fill (+ st) gives the bits of the arm filling itself, and
    keep_cache=False gives the same logits with the late caches dropped.
Bars: 1e-2 relative Frobenius on logits, on the filled GDN states (taken through fill_store right after the
fill) and on K / V; 2e-2 on the GDN states after the tail has run through every late layer (each layer's
tail input is the previous layer's output, so those states carry the earlier layers' rounding differences
too); argmax agreement > 0.9; reuse bitwise, and a reusing arm's caches stay its own."""
import numpy as np
import pytest
import torch

import gguf_writer
from fill_cases import case, hybrid_config, hybrid_tensors, inputs, rel_err
from oracle import kva as OK
from oracle import model as OM

pytestmark = pytest.mark.gpu
TOL = 1e-2
SPLIT, N, TAIL, KEEP = 4, 900, 192, 64


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.fixture(scope="module")
def hybrid():
    cfg = hybrid_config(["gdn", "gdn", "gdn", "attn"] * 2)
    return cfg, hybrid_tensors(cfg, seed=9)


def _write_adapter(path, cfg, rng):
    """An adapter for layers 4..7 of the hybrid: an F16 map and F32 bias for attention layer 7, F32 st
    corrections [heads, V, K] for GDN layers 4..6 (no maps: the engine feeds them h_S)."""
    H, nv = cfg["hidden_size"], cfg["linear_num_value_heads"]
    kinds = " ".join(cfg["layer_types"])
    meta = [("general.architecture", "str", "qwen35"), ("adapter.ridgefill.split", "u32", SPLIT),
            ("adapter.ridgefill.n_embd", "u32", H), ("adapter.ridgefill.model_layer_types", "str", kinds)]
    w7 = (np.eye(H) + 0.05 * rng.standard_normal((H, H)) / H ** 0.5).astype(np.float16)
    b7 = (0.01 * rng.standard_normal(H)).astype(np.float32)
    st = {L: (0.01 * rng.standard_normal((nv, 128, 128))).astype(np.float32) for L in (4, 5, 6)}
    tensors = [(f"blk.{L}.ridgefill.st", (128, 128, nv), 0, st[L].tobytes()) for L in (4, 5, 6)]
    tensors += [("blk.7.ridgefill.weight", (H, H), 1, w7.tobytes()), ("blk.7.ridgefill.bias", (H,), 0, b7.tobytes())]
    gguf_writer.write(path, meta, tensors)
    W = {7: torch.from_numpy(w7.astype(np.float32)).to(torch.bfloat16)}
    B = {7: torch.from_numpy(b7).to(torch.bfloat16)}
    return W, B, {L: torch.from_numpy(st[L]).transpose(1, 2).contiguous() for L in st}


def _compare(cache, oc, logits, want, layers, types, stored=None, ostored=None):
    """(logits, filled GDN states, K / V, argmax agreement, GDN states after the tail) errors."""
    el = rel_err(logits, want)
    gdn = [i for i in layers if types[i] == "gdn"]
    es_tail = max([rel_err(cache[i]["rec"], oc[i]["rec"]) for i in gdn] or [0.0])
    es = max([rel_err(stored[i]["rec"], ostored[i]["rec"]) for i in gdn] or [0.0]) if stored is not None else es_tail
    ek = max([rel_err(cache[i][p], oc[i][p]) for i in layers if types[i] == "attn" for p in ("k", "v")] or [0.0])
    agree = float((logits.argmax(-1).cpu() == want.argmax(-1)).float().mean())
    return el, es, ek, agree, es_tail


@pytest.mark.parametrize("exact", [False, True])
def test_gguf_adapter_drives_hybrid_finish(dev, hybrid, tmp_path, exact):
    from rfill.kva import adapter_arm, finish, load_gguf
    from rfill.model import FillModel
    cfg, t = hybrid
    W, B, st = _write_adapter(tmp_path / "ad.gguf", cfg, np.random.default_rng(3))
    proj = load_gguf(tmp_path / "ad.gguf", device=dev)
    arm = adapter_arm("kva+st", proj, TAIL)
    assert arm.fill == "by_type" and arm.fill_of("gdn") == "identity" and sorted(arm.st) == [4, 5, 6]
    h = inputs(N, cfg["hidden_size"], seed=61)
    P = N - TAIL
    g = torch.Generator().manual_seed(62)
    rows = torch.randperm(P, generator=g)[:10].sort().values if exact else None
    m = FillModel(cfg, t, dev)
    ids = torch.zeros(N, dtype=torch.long)
    stored, ostored = {}, {}
    logits, cache, P_got = finish(m, ids, h, None, arm, KEEP, exact_rows=rows, fill_store=stored)
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oarm = OK.Arm("kva+st", split=SPLIT, tail=TAIL, fill="by_type", projector=OK.Projector(SPLIT, W, B), st=st,
                  fill_by_type={"attention": "proj", "gdn": "identity"})
    want, oc, P_want = OK.finish(om, ids, h, om.new_cache(), oarm, KEEP, exact_rows=rows, fill_store=ostored)
    assert P_got == P_want == P
    el, es, ek, agree, es_tail = _compare(cache, oc, logits, want, range(SPLIT, 8), m.layer_types, stored, ostored)
    print(f"adapter by_type finish (exact rows: {exact}): logits {el:.2e}, filled GDN states {es:.2e} "
          f"(after the tail {es_tail:.2e}), K/V {ek:.2e}, argmax {agree:.3f}")
    assert el < TOL and es < TOL and es_tail < 2 * TOL and ek < TOL and agree > 0.9


def test_kvexact_hybrid_arm(dev, hybrid):
    """{'attention': 'oracle', 'gdn': 'proj'} (the reference's kvexact kind): attention layers filled from
    given true inputs, GDN layers from the projector."""
    from rfill.kva import Arm, Projector, finish
    from rfill.model import FillModel
    cfg, t = hybrid
    H = cfg["hidden_size"]
    h = inputs(N, H, seed=63)
    g = torch.Generator().manual_seed(64)
    W = {i: (torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16) for i in (4, 5, 6)}
    B = {i: (1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for i in (4, 5, 6)}
    true = {i: inputs(N, H, seed=70 + i) for i in range(SPLIT, 8)}
    by = {"attention": "oracle", "gdn": "proj"}
    m = FillModel(cfg, t, dev)
    ids = torch.zeros(N, dtype=torch.long)
    arm = Arm("kvexact", split=SPLIT, tail=TAIL, fill="by_type", fill_by_type=by, projector=Projector(SPLIT, W, B))
    stored, ostored = {}, {}
    logits, cache, _ = finish(m, ids, h, None, arm, KEEP, oracle={i: x.to(dev) for i, x in true.items()},
                              fill_store=stored)
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oarm = OK.Arm("kvexact", split=SPLIT, tail=TAIL, fill="by_type", fill_by_type=by, projector=OK.Projector(SPLIT, W, B))
    want, oc, _ = OK.finish(om, ids, h, om.new_cache(), oarm, KEEP, oracle=true, fill_store=ostored)
    el, es, ek, agree, es_tail = _compare(cache, oc, logits, want, range(SPLIT, 8), m.layer_types, stored, ostored)
    print(f"kvexact finish: logits {el:.2e}, filled GDN states {es:.2e} (after the tail {es_tail:.2e}), K/V {ek:.2e}, "
          f"argmax {agree:.3f}")
    assert el < TOL and es < TOL and es_tail < 2 * TOL and ek < TOL and agree > 0.9
    with pytest.raises(ValueError, match="oracle"):
        finish(m, ids, h, None, arm, KEEP)                  # an oracle fill needs the true inputs


def test_none_fill_with_exact_rows(dev):
    """fill 'none' (skip + select): only the exact rows run each late layer, over themselves; then the tail."""
    from rfill.kva import Arm, finish
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=8)
    H, P = cfg["hidden_size"], 2048 - 256
    h = inputs(2048, H, seed=65)
    g = torch.Generator().manual_seed(66)
    rows = torch.randperm(P, generator=g)[:40].sort().values
    m = FillModel(cfg, t, dev)
    ids = torch.zeros(2048, dtype=torch.long)
    logits, cache, _ = finish(m, ids, h, None, Arm("skip", split=5, tail=256, fill="none"), 100, exact_rows=rows)
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    want, oc, _ = OK.finish(om, ids, h, om.new_cache(), OK.Arm("skip", split=5, tail=256, fill="none"), 100,
                            exact_rows=rows)
    for i in range(5, 8):
        assert cache[i]["n"] == oc[i]["n"] == 40 + 256
    el, _, ek, agree, _ = _compare(cache, oc, logits, want, range(5, 8), m.layer_types)
    print(f"fill 'none' with 40 exact rows: logits {el:.2e}, K/V {ek:.2e}, argmax {agree:.3f}")
    assert el < TOL and ek < TOL and agree > 0.9


def test_fill_reuse_and_keep_cache(dev, hybrid):
    """A base arm stores its fill; an arm with the same fill plus st reuses it (fill_reuse) and gives the bits of
    the same arm filling itself; keep_cache=False drops the late caches and keeps the logits."""
    from rfill.kva import Arm, Projector, finish
    from rfill.model import FillModel
    cfg, t = hybrid
    H = cfg["hidden_size"]
    h = inputs(N, H, seed=67).to(dev)
    g = torch.Generator().manual_seed(68)
    W = {i: (torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16) for i in range(4, 8)}
    B = {i: (1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for i in range(4, 8)}
    st = {i: (0.01 * torch.randn(4, 128, 128, generator=g)).to(dev) for i in (4, 5, 6)}
    proj = Projector(SPLIT, W, B)
    m = FillModel(cfg, t, dev)
    ids = torch.zeros(N, dtype=torch.long)
    store = {}
    base, _, _ = finish(m, ids, h, None, Arm("kva", split=SPLIT, tail=TAIL, fill="proj", projector=proj), KEEP,
                        fill_store=store)
    plus = Arm("kva+st", split=SPLIT, tail=TAIL, fill="proj", projector=proj, st=st)
    fresh, c1, _ = finish(m, ids, h, None, plus, KEEP)
    reused, c2, _ = finish(m, ids, h, None, plus, KEEP, fill_reuse=store)
    dropped, c3, _ = finish(m, ids, h, None, plus, KEEP, fill_reuse=store, keep_cache=False)
    again, _, _ = finish(m, ids, h, None, Arm("kva", split=SPLIT, tail=TAIL, fill="proj", projector=proj), KEEP,
                         fill_reuse=store)
    torch.cuda.synchronize()
    assert sorted(store) == list(range(SPLIT, 8)) and store[7]["n"] == N - TAIL
    assert torch.equal(fresh, reused) and torch.equal(reused, dropped) and torch.equal(base, again)
    assert not torch.equal(base, fresh)                     # st changes the tail
    assert all(c3[i] == {} for i in range(SPLIT, 8)) and c2[7]["n"] == N
    # the reusing arm's caches are its own: later arms reusing the same fill did not write into them
    assert torch.equal(c1[7]["k"], c2[7]["k"]) and torch.equal(c1[7]["v"], c2[7]["v"])
    assert torch.equal(c1[4]["rec"], c2[4]["rec"]) and c2[7]["kbuf"].data_ptr() != store[7]["kbuf"].data_ptr()
    assert torch.equal(store[7]["k"], c1[7]["k"][:, :N - TAIL])            # the stored fill is intact
    with pytest.raises(ValueError, match="fill reuse"):
        finish(m, ids, h, None, plus, KEEP, fill_reuse=store, exact_rows=[3, 5])
