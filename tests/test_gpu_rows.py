"""GPU parity of the exact rows' full layer (FillModel.layer_rows: rf_row_gather, rf_norm_q, rf_attend_rows,
rf_residual_add, rf_silu_mul over rf_map_apply / rf_norm_linear) against the CPU oracle's layer_rows
(code/kva/model.py:259-276) and of the attention kernel against the oracle's attend_at
(code/kva/ops.py:131-155) on identical seeded inputs.

Bars: outputs within relative Frobenius error 1e-2 (bf16 path); the filled cache as in the fill tests;
causality: keys after a query's position never change its output (bitwise), keys before it do."""
import pytest
import torch

from fill_cases import case, inputs, rel_err
from oracle import model as OM
from oracle import ops as oops

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _qkv(nq, hq, hkv, d, n, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(nq, hq * d, generator=g).to(torch.bfloat16)
    k = torch.randn(hkv, n, d, generator=g).to(torch.bfloat16)
    v = torch.randn(hkv, n, d, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (4, 2, 64), (8, 8, 128), (16, 2, 64)])
def test_attend_rows_matches_oracle(dev, hq, hkv, d):
    from rfill import ops
    n, nq = 1500, 70
    q, k, v = _qkv(nq, hq, hkv, d, n, seed=hq + d)
    g = torch.Generator().manual_seed(5)
    qpos = torch.randperm(n, generator=g)[:nq].sort().values
    qpos[0], qpos[-1] = 0, n - 1                      # a query that sees one key, one that sees them all
    qpos = qpos.sort().values
    kb = torch.zeros(hkv, n + 64, d, dtype=torch.bfloat16)
    vb = torch.zeros_like(kb)
    kb[:, :n], vb[:, :n] = k, v
    scale = d ** -0.5
    got = ops.attend_rows(q.to(dev), qpos.to(dev), kb.to(dev), vb.to(dev), n, hq, scale)          # key splits
    one = ops.attend_rows(q.to(dev), qpos.to(dev), kb.to(dev), vb.to(dev), n, hq, scale, workspace=None)
    torch.cuda.synchronize()
    want = oops.attend_at(q.view(nq, hq, d).transpose(0, 1), k, v, scale, qpos)
    err, err1 = rel_err(got, want), rel_err(one, want)
    print(f"hq {hq} hkv {hkv} d {d}: attention rel err {err:.2e} (split keys), {err1:.2e} (one pass)")
    assert err < TOL and err1 < TOL
    assert ops.attend_rows_workspace_bytes(nq, hq, hkv, d, n) > 0
    # the query at position 0 sees only key 0: its output is V[0] of its K / V head exactly (p = 1)
    rep = hq // hkv
    for res in (got, one):
        first = res[0].view(hq, d).cpu()
        for h in range(hq):
            assert torch.equal(first[h], v[h // rep, 0])


def test_attend_rows_is_causal(dev):
    """Keys after every query's position leave the outputs bitwise unchanged; a key before changes them."""
    from rfill import ops
    hq, hkv, d, n, nq = 32, 8, 128, 900, 20
    q, k, v = _qkv(nq, hq, hkv, d, n, seed=3)
    qpos = torch.arange(nq) * 20 + 5                  # max position 385 < n
    kb = torch.zeros(hkv, n + 64, d, dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    kb[:, :n], vb[:, :n] = k.to(dev), v.to(dev)
    for ws in ("auto", None):
        base = ops.attend_rows(q.to(dev), qpos.to(dev), kb, vb, n, hq, d ** -0.5, workspace=ws)
        again = ops.attend_rows(q.to(dev), qpos.to(dev), kb, vb, n, hq, d ** -0.5, workspace=ws)
        assert torch.equal(base, again)                   # run to run, the same bits
        kb2, vb2 = kb.clone(), vb.clone()
        kb2[:, 400:n] = 7.0
        vb2[:, 400:n] = -3.0
        later = ops.attend_rows(q.to(dev), qpos.to(dev), kb2, vb2, n, hq, d ** -0.5, workspace=ws)
        assert torch.equal(base, later)
        vb2[:, 0] += 1.0
        earlier = ops.attend_rows(q.to(dev), qpos.to(dev), kb2, vb2, n, hq, d ** -0.5, workspace=ws)
        assert not torch.equal(base, earlier)


@pytest.mark.parametrize("name", ["llama_c1", "llama3_scaled", "qwen3_knorm"])
def test_layer_rows_matches_oracle(dev, name):
    from rfill.model import FillModel
    cfg, t = case(name)
    P, H = 1200, cfg["hidden_size"]
    x = inputs(P, H, seed=21)
    g = torch.Generator().manual_seed(22)
    rows = torch.randperm(P, generator=g)[:37].sort().values
    rows[0] = 0
    rows = rows.sort().values.unique()
    pos = torch.arange(P)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    want = om.layer_rows(0, x, pos, rows, oc)
    m = FillModel(cfg, t, dev)
    c = m.new_cache()
    got = m.layer_rows(0, x.to(dev), pos.to(dev), rows.to(dev), c)
    torch.cuda.synchronize()
    err = rel_err(got, want)
    ek, ev = rel_err(c[0]["k"], oc[0]["k"]), rel_err(c[0]["v"], oc[0]["v"])
    # the layer's own contribution (output minus input), the part an error would hide in
    ed = rel_err(got.cpu().float() - x[rows].float(), want.float() - x[rows].float())
    print(f"{name}: layer_rows out rel err {err:.2e}, update {ed:.2e}, K {ek:.2e}, V {ev:.2e}")
    assert err < TOL and ed < TOL and ek < TOL and ev < TOL
    assert c[0]["n"] == P


def test_layer_rows_refuses_a_filled_cache(dev):
    from rfill.model import FillModel
    from fill_cases import gdn_config, gdn_tensors
    cfg, t = case("llama_c1")
    m = FillModel(cfg, t, dev)
    x = inputs(300, cfg["hidden_size"], seed=2).to(dev)
    pos = torch.arange(300, device=dev)
    c = m.new_cache()
    m.fill(0, x, pos, c)
    with pytest.raises(ValueError):
        m.layer_rows(0, x, pos, torch.tensor([3, 9], device=dev), c)
    gcfg = gdn_config()
    gm = FillModel(gcfg, gdn_tensors(gcfg), dev)
    gx = inputs(64, gcfg["hidden_size"]).to(dev)
    gc = gm.new_cache()
    gm.fill(0, gx, torch.arange(64, device=dev), gc)
    with pytest.raises(ValueError):                               # a GDN layer's filled state
        gm.layer_rows(0, gx, torch.arange(64, device=dev), torch.tensor([1], device=dev), gc)


def test_fill_late_runs_the_exact_rows_through_every_layer(dev):
    """finish()'s late loop with exact rows and no given inputs: the rows start from h_split and each late
    layer's layer_rows gives their next input; caches and row inputs against the oracle's finish loop."""
    from rfill.kva import Arm, Projector, fill_late
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=8)
    N, tail, split = 2048, 256, 5
    P, H = N - tail, cfg["hidden_size"]
    h = inputs(N, H, seed=12)
    g = torch.Generator().manual_seed(13)
    W = {i: (torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16)
         for i in range(split, 8)}
    B = {i: (1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for i in range(split, 8)}
    rows = torch.randperm(P, generator=g)[:18].sort().values
    arm = Arm("ridgefill", split=split, tail=tail, fill="proj", projector=Projector(split, W, B))
    m = FillModel(cfg, t, dev)
    got_inputs = {}
    cache, P_got = fill_late(m, h.to(dev), arm, exact_rows=rows, row_inputs=got_inputs)
    torch.cuda.synchronize()
    assert P_got == P
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    pos = torch.arange(P)
    hr = h[rows]
    for i in range(split, 8):
        eh = rel_err(got_inputs[i], hr)
        x = torch.nn.functional.linear(h[:P], W[i], B[i]).index_copy(0, rows, hr)
        hr = om.layer_rows(i, x, pos, rows, oc)
        ek, ev = rel_err(cache[i]["k"], oc[i]["k"]), rel_err(cache[i]["v"], oc[i]["v"])
        er = rel_err(cache[i]["k"][:, rows.to(dev)], oc[i]["k"][:, rows])
        print(f"layer {i}: row inputs {eh:.2e}, K {ek:.2e} V {ev:.2e} exact-row K {er:.2e}")
        assert eh < TOL and ek < TOL and ev < TOL and er < TOL


@pytest.mark.parametrize("hq,hkv,d,nq,slot0,n", [(32, 8, 128, 300, 1000, 1300),      # a tail: the last nq keys
                                                 (8, 8, 64, 700, 0, 700),             # group 1, from slot 0
                                                 (16, 2, 128, 333, 517, 1200),        # group 8, keys after
                                                 (4, 2, 64, 1000, 90, 1100),          # group 2, partial block
                                                 (32, 8, 128, 64, 5, 69),             # fewer keys than a tile pair
                                                 (16, 2, 256, 300, 1000, 1300),       # d 256, group 8: a tail
                                                 (4, 4, 256, 200, 0, 200),            # d 256, group 1, slot 0
                                                 (16, 1, 256, 100, 50, 400),          # d 256, group 16
                                                 (16, 2, 256, 40, 5, 45)])            # d 256, one partial tile
def test_attend_causal_matches_oracle(dev, hq, hkv, d, nq, slot0, n):
    """The many-query kernel (rf_attend_causal: V read transposed out of LDS, 256 query rows per block)
    against the oracle's attend_at at positions slot0 .. slot0 + nq - 1 (attend itself when they are the
    last keys), and against rf_attend_rows on the same queries."""
    from rfill import ops
    q, k, v = _qkv(nq, hq, hkv, d, n, seed=nq + d)
    cap = n + 64
    kb = torch.zeros(hkv, cap, d, dtype=torch.bfloat16)
    vb = torch.zeros_like(kb)
    kb[:, :n], vb[:, :n] = k, v
    vb[:, n:] = float("nan")                          # rows past the keys must never be read
    scale = d ** -0.5
    qd, kd, vd = q.to(dev), kb.to(dev), vb.to(dev)
    got = ops.attend_causal(qd, slot0, kd, vd, n, hq, scale)
    qpos = torch.arange(slot0, slot0 + nq)
    rows = ops.attend_rows(qd, qpos.to(dev), kd, vd, n, hq, scale)
    torch.cuda.synchronize()
    qh = q.view(nq, hq, d).transpose(0, 1)
    want = (oops.attend(qh, k, v, scale) if slot0 + nq == n
            else oops.attend_at(qh, k, v, scale, qpos))
    err, err_rows = rel_err(got, want), rel_err(got, rows)
    print(f"hq {hq} hkv {hkv} d {d} nq {nq} slot0 {slot0} n {n}: rel err {err:.2e} vs oracle, "
          f"{err_rows:.2e} vs rf_attend_rows")
    assert torch.isfinite(got.float()).all()
    assert err < TOL and err_rows < TOL
    if slot0 == 0:                                    # the query at slot 0 sees key 0 only: V[0] exactly
        first = got[0].view(hq, d).cpu()
        for h in range(hq):
            assert torch.equal(first[h], v[h // (hq // hkv), 0])


def test_attend_causal_is_causal_and_deterministic(dev):
    from rfill import ops
    hq, hkv, d, n, nq = 32, 8, 128, 900, 300
    q, k, v = _qkv(nq, hq, hkv, d, n, seed=7)
    kb = torch.zeros(hkv, n + 64, d, dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    kb[:, :n], vb[:, :n] = k.to(dev), v.to(dev)
    slot0 = 400                                       # queries at slots 400 .. 699; keys 700 .. 899 unseen
    base = ops.attend_causal(q.to(dev), slot0, kb, vb, n, hq, d ** -0.5)
    again = ops.attend_causal(q.to(dev), slot0, kb, vb, n, hq, d ** -0.5)
    assert torch.equal(base, again)
    kb2, vb2 = kb.clone(), vb.clone()
    kb2[:, 700:n] = 7.0
    vb2[:, 700:n] = -3.0
    assert torch.equal(base, ops.attend_causal(q.to(dev), slot0, kb2, vb2, n, hq, d ** -0.5))
    # a key between the first and the last query changes only the queries at or after it
    vb2[:, 550] += 1.0
    later = ops.attend_causal(q.to(dev), slot0, kb2, vb2, n, hq, d ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(base[:150], later[:150])
    assert not torch.equal(base[150:], later[150:])


def test_attend_causal_refuses(dev):
    from rfill import ops
    kb = torch.zeros(2, 200, 128, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(10, 4 * 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.attend_causal(q, 195, kb, kb.clone(), 200, 4, 0.1)                # slots past the keys
    q6 = torch.zeros(10, 6 * 128, dtype=torch.bfloat16, device=dev)
    from rfill._lib import UnsupportedArchitecture
    with pytest.raises(UnsupportedArchitecture):
        ops.attend_causal(q6, 0, kb, kb.clone(), 200, 6, 0.1)                 # group of 3


@pytest.mark.parametrize("hq,hkv,d,nq,n", [(32, 8, 128, 150, 6000), (16, 2, 128, 37, 3000), (4, 2, 64, 300, 2500),
                                           (8, 8, 64, 5, 900), (16, 2, 256, 150, 3000), (8, 2, 256, 37, 2000)])
def test_attend_causal_at_positions(dev, hq, hkv, d, nq, n):
    """rf_attend_causal with sorted query positions (the exact rows' attention): with the key range split
    over blocks (full workspace) and unsplit (a workspace holding only V transposed), against the oracle's
    attend_at and rf_attend_rows; split results the same bits run to run."""
    from rfill import ops
    q, k, v = _qkv(nq, hq, hkv, d, n, seed=nq + n)
    g = torch.Generator().manual_seed(nq)
    qpos = torch.randperm(n, generator=g)[:nq].sort().values
    qpos[0] = 0                                        # a query that sees only key 0
    qpos = qpos.sort().values.unique()
    q = q[:qpos.shape[0]]
    nq = q.shape[0]
    kb = torch.zeros(hkv, n + 64, d, dtype=torch.bfloat16)
    vb = torch.zeros_like(kb)
    kb[:, :n], vb[:, :n] = k, v
    vb[:, n:] = float("nan")
    scale = d ** -0.5
    qd, kd, vd, pd = q.to(dev), kb.to(dev), vb.to(dev), qpos.to(dev)
    full = ops.attend_causal_workspace_bytes(nq, hq, hkv, d, n)
    vt_only = hkv * d * ((n + 63) // 64 * 64) * 2
    vt_only = (vt_only + 255) // 256 * 256
    assert full > vt_only                              # these sizes split the key range
    split = ops.attend_causal(qd, 0, kd, vd, n, hq, scale, qpos=pd)
    again = ops.attend_causal(qd, 0, kd, vd, n, hq, scale, qpos=pd)
    one = ops.attend_causal(qd, 0, kd, vd, n, hq, scale, qpos=pd,
                            workspace=torch.empty(vt_only, dtype=torch.uint8, device=dev))
    rows = ops.attend_rows(qd, pd, kd, vd, n, hq, scale)
    torch.cuda.synchronize()
    want = oops.attend_at(q.view(nq, hq, d).transpose(0, 1), k, v, scale, qpos)
    e_s, e_1, e_r = rel_err(split, want), rel_err(one, want), rel_err(split, rows)
    print(f"hq {hq} hkv {hkv} d {d} nq {nq} n {n}: split {e_s:.2e}, one pass {e_1:.2e} vs oracle; "
          f"{e_r:.2e} vs rf_attend_rows")
    assert torch.isfinite(split.float()).all() and torch.isfinite(one.float()).all()
    assert e_s < TOL and e_1 < TOL and e_r < TOL
    assert torch.equal(split, again)
    first = split[0].view(hq, d).cpu()
    for h in range(hq):
        assert torch.equal(first[h], v[h // (hq // hkv), 0])


def test_attend_rows_head_dim_256_many_queries(dev):
    """An exact tail at head_dim 256 (Qwen3.5's gated attention): 2600 queries take the 512-thread,
    128-row-block variant; against the oracle's attend_at and bitwise against the 64-row variant run over
    the same queries in pieces of fewer than 2048 (no key-range splits in either)."""
    from oracle import ops as oops
    from rfill import ops
    hq, hkv, d, n, nq = 16, 2, 256, 4000, 2600
    q, k, v = _qkv(nq, hq, hkv, d, n, seed=77)
    qpos = torch.arange(n - nq, n)
    kb = torch.zeros(hkv, n + 64, d, dtype=torch.bfloat16)
    vb = torch.zeros_like(kb)
    kb[:, :n], vb[:, :n] = k, v
    kb, vb, qd, pd = kb.to(dev), vb.to(dev), q.to(dev), qpos.to(dev)
    scale = d ** -0.5
    wide = ops.attend_rows(qd, pd, kb, vb, n, hq, scale, workspace=None)
    parts = torch.cat([ops.attend_rows(qd[a:b], pd[a:b], kb, vb, n, hq, scale, workspace=None)
                       for a, b in ((0, 1300), (1300, 2600))])
    torch.cuda.synchronize()
    assert torch.equal(wide, parts)
    want = oops.attend_at(q.view(nq, hq, d).transpose(0, 1), k, v, scale, qpos)
    err = rel_err(wide, want)
    print(f"head_dim 256, {nq} queries: rel err {err:.2e}")
    assert err < TOL


@pytest.mark.parametrize("R,knorm", [(287, True), (700, False)])
def test_norm_kv_rows_writes_each_row_at_its_slot(dev, R, knorm):
    """rf_norm_kv_rows: row j's K / V, normed, projected, k_normed and rotated at position rows[j], land in
    slot rows[j] and nowhere else; bit-identical to rf_norm_kv_write of the same rows at slots 0.. with the
    gathered RoPE table, chunk by chunk of at most 512 rows (both take the few-rows partials then)."""
    from rfill import ops
    H, hkv, d, P = 1024, 2, 128, 3000
    g = torch.Generator().manual_seed(R)
    rows = torch.randperm(P, generator=g)[:R].sort().values.to(dev)
    x = (torch.randn(R, H, generator=g)).to(torch.bfloat16).to(dev)
    ssq = ops.row_ssq(x)
    wkv = (torch.randn(2 * hkv * d, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    kn = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev) if knorm else None
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    cs = ops.rope_table(torch.arange(P, device=dev), inv.to(dev))
    kb, vb = (torch.zeros(hkv, P, d, dtype=torch.bfloat16, device=dev) for _ in range(2))
    ops.norm_kv_rows(x, ssq, 1e-6, wkv, hkv, d, kn, 0, cs, rows, kb, vb)
    want_k, want_v = (torch.zeros(hkv, R, d, dtype=torch.bfloat16, device=dev) for _ in range(2))
    for r0 in range(0, R, 512):
        r1 = min(R, r0 + 512)
        csr = cs[rows[r0:r1]].contiguous()
        ops.norm_kv_write(x[r0:r1], ssq[r0:r1], 1e-6, wkv, hkv, d, kn, 0, csr, want_k, want_v, r0, workspace="auto")
    torch.cuda.synchronize()
    assert torch.equal(kb[:, rows], want_k) and torch.equal(vb[:, rows], want_v)
    rest = torch.ones(P, dtype=torch.bool, device=dev)
    rest[rows] = False
    assert not kb[:, rest].any() and not vb[:, rest].any()
    with pytest.raises(ValueError, match="beyond the cache"):
        ops.norm_kv_rows(x, ssq, 1e-6, wkv, hkv, d, kn, 0, cs, rows, kb[:, :100], vb[:, :100])


@pytest.mark.parametrize("R,norms", [(287, True), (600, False)])
def test_norm_qkv_rows_matches_the_separate_products(dev, R, norms):
    """rf_norm_qkv_rows: queries as rf_norm_q and the rows' K / V at slots pos as rf_norm_kv_rows, from one
    product over [wq; wkv] (its K split differs, so the bf16 results agree to rounding); slots other than
    the rows' stay untouched."""
    from rfill import ops
    H, hq, hkv, d, P = 1024, 8, 2, 128, 3000
    g = torch.Generator().manual_seed(R + 1)
    rows = torch.randperm(P, generator=g)[:R].sort().values.to(dev)
    x = torch.randn(R, H, generator=g).to(torch.bfloat16).to(dev)
    ssq = ops.row_ssq(x)
    wqkv = (torch.randn((hq + 2 * hkv) * d, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    qn = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev) if norms else None
    kn = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev) if norms else None
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    cs = ops.rope_table(torch.arange(P, device=dev), inv.to(dev))
    kb, vb, kb2, vb2 = (torch.zeros(hkv, P, d, dtype=torch.bfloat16, device=dev) for _ in range(4))
    q = ops.norm_qkv_rows(x, ssq, 1e-6, wqkv, hq, hkv, d, qn, kn, 0, cs, rows, kb, vb)
    q2 = ops.norm_q(x, ssq, 1e-6, wqkv[:hq * d].contiguous(), hq, d, qn, 0, cs, rows, workspace="auto")
    ops.norm_kv_rows(x, ssq, 1e-6, wqkv[hq * d:].contiguous(), hkv, d, kn, 0, cs, rows, kb2, vb2)
    torch.cuda.synchronize()
    for got, want in ((q, q2), (kb[:, rows], kb2[:, rows]), (vb[:, rows], vb2[:, rows])):
        assert rel_err(got, want) < 5e-3
    rest = torch.ones(P, dtype=torch.bool, device=dev)
    rest[rows] = False
    assert not kb[:, rest].any() and not vb[:, rest].any()


def test_rows_workspace_covers_a_short_last_chunk(dev):
    """655 rows of a Qwen3-8B-width [wq; wkv] product (H 4096, 32 query / 8 KV heads: N 6144): the last
    chunk of 143 rows splits K 8 ways (28.1 MB of partials) against 2 ways for the first 512 rows (25.2 MB).
    With the workspace rf_rows_workspace_bytes gives, a guard region right after it stays untouched and the
    results match the separate products; a workspace sized for the first chunk only is refused."""
    from rfill import ops
    H, hq, hkv, d, P, R = 4096, 32, 8, 128, 4000, 655
    g = torch.Generator().manual_seed(655)
    rows = torch.randperm(P, generator=g)[:R].sort().values.to(dev)
    x = torch.randn(R, H, generator=g).to(torch.bfloat16).to(dev)
    ssq = ops.row_ssq(x)
    wqkv = (torch.randn((hq + 2 * hkv) * d, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    kn = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    cs = ops.rope_table(torch.arange(P, device=dev), inv.to(dev))
    need = ops.rows_workspace_bytes(R, (hq + 2 * hkv) * d, H)
    assert need == 8 * 143 * 6144 * 4
    guard = 1 << 20
    buf = torch.full((need + guard,), 0xA5, dtype=torch.uint8, device=dev)
    kb, vb, kb2, vb2 = (torch.zeros(hkv, P, d, dtype=torch.bfloat16, device=dev) for _ in range(4))
    q = ops.norm_qkv_rows(x, ssq, 1e-6, wqkv, hq, hkv, d, None, kn, 0, cs, rows, kb, vb, workspace=buf[:need])
    q2 = ops.norm_q(x, ssq, 1e-6, wqkv[:hq * d].contiguous(), hq, d, None, 0, cs, rows, workspace="auto")
    ops.norm_kv_rows(x, ssq, 1e-6, wqkv[hq * d:].contiguous(), hkv, d, kn, 0, cs, rows, kb2, vb2)
    torch.cuda.synchronize()
    assert bool((buf[need:] == 0xA5).all()), "write past the workspace"
    for got, want in ((q, q2), (kb[:, rows], kb2[:, rows]), (vb[:, rows], vb2[:, rows])):
        assert rel_err(got, want) < 5e-3
    short = ops.gemm_workspace_bytes(512, (hq + 2 * hkv) * d, H)
    assert short < need
    with pytest.raises(ValueError, match="workspace"):
        ops.norm_qkv_rows(x, ssq, 1e-6, wqkv, hq, hkv, d, None, kn, 0, cs, rows, kb, vb, workspace=buf[:short])


def test_rows_positions_outside_the_cache_are_skipped(dev):
    """With pos_max given the positions are not read back; rows whose position lies outside the cache view
    or the table (here 120 and -3 for a 100-slot view) are skipped on the device. The view sits inside a
    larger buffer, so a write past either end of it would show; the kept rows are bit-identical to a call
    over the kept rows alone."""
    from rfill import ops
    H, hkv, d = 1024, 2, 128
    g = torch.Generator().manual_seed(3)
    pos = torch.tensor([5, 50, 120, -3, 99], dtype=torch.int64, device=dev)
    keep = torch.tensor([0, 1, 4], device=dev)
    x = torch.randn(5, H, generator=g).to(torch.bfloat16).to(dev)
    ssq = ops.row_ssq(x)
    wkv = (torch.randn(2 * hkv * d, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    cs_all = ops.rope_table(torch.arange(300, device=dev), inv.to(dev))
    cs = cs_all[100:200]
    kb_all, vb_all, kb2, vb2 = (torch.zeros(hkv, 300, d, dtype=torch.bfloat16, device=dev) for _ in range(4))
    ops.norm_kv_rows(x, ssq, 1e-6, wkv, hkv, d, None, 0, cs, pos, kb_all[:, 100:200], vb_all[:, 100:200], pos_max=99)
    ops.norm_kv_rows(x[keep].contiguous(), ssq[keep].contiguous(), 1e-6, wkv, hkv, d, None, 0, cs, pos[keep],
                     kb2[:, 100:200], vb2[:, 100:200], pos_max=99)
    torch.cuda.synchronize()
    assert torch.equal(kb_all, kb2) and torch.equal(vb_all, vb2)
    written = kb_all.abs().sum(dim=(0, 2)).nonzero().flatten().tolist()
    assert written == [105, 150, 199]


@pytest.mark.parametrize("R", [287, 1300])
def test_fused_residual_and_swiglu_epilogues_are_bit_identical(dev, R):
    """map_apply_residual == map_apply + residual_add and norm_linear_swiglu == norm_linear + silu_mul, bit
    for bit, with every row in the split sums' epilogue (287 rows) and through the unsplit kernels (1300)."""
    from rfill import ops
    H, I = 1024, 1536
    g = torch.Generator().manual_seed(R + 7)
    x = torch.randn(R, H, generator=g).to(torch.bfloat16).to(dev)
    res = torch.randn(R, H, generator=g).to(torch.bfloat16).to(dev)
    wo = (torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    wgu = (torch.randn(2 * I, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    ws = lambda n, k: torch.empty(max(1, ops.gemm_workspace_bytes(R, n, k)), dtype=torch.uint8, device=dev)  # noqa: E731
    h1, s1 = ops.map_apply_residual(x, wo, res, workspace=ws(H, H))
    a, _ = ops.map_apply(x, wo, None, workspace=ws(H, H))
    want_h1, want_s1 = ops.residual_add(res, a)
    act = ops.norm_linear_swiglu(h1, s1, 1e-5, wgu, workspace=ws(2 * I, H))
    want_act = ops.silu_mul(ops.norm_linear(want_h1, want_s1, 1e-5, wgu, workspace=ws(2 * I, H)))
    torch.cuda.synchronize()
    assert torch.equal(h1, want_h1) and torch.equal(s1, want_s1)
    assert torch.equal(act, want_act)
