"""GPU tests of the batched fill launches (rf_map_apply_batch, rf_norm_kv_write_batch: the maps and the
K / V fills of several late layers in one launch each, on persistent tiles) and of fill_late's grouped
schedule.

Bar: bitwise. Every layer's x, row statistics and K / V cache equal the per-layer launches' without a
split-K workspace (the same tiles, the same MFMA order, the same epilogue arithmetic); cache slots outside
the written rows keep their contents. The per-layer launches themselves are pinned to the oracle in
test_gpu_fill.py."""
import pytest
import torch

from fill_cases import CASES, attn_config, case, inputs, random_tensors, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _maps(H, layers, seed):
    g = torch.Generator().manual_seed(seed)
    W = [(torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16) for _ in layers]
    B = [(1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for _ in layers]
    return W, B


# Width-1024 configurations take the persistent K / V kernel (the CASES widths 256 / 512 take the per-tile
# kernel): its d-128 K epilogue without and with k_norm, and the generic one (d 256 with rot 64, d 64, and
# rot 8, whose table row is a single 16-byte chunk).
WIDE = {
    "w1024_llama_d128": ("llama", 1024, 2, 128, 5e5, {}),
    "w1024_qwen3_knorm": ("qwen3", 1024, 2, 128, 1e6, dict(eps=1e-6)),
    "w1024_qwen35_d256_rot64": ("qwen3_5", 1024, 2, 256, 1e7, dict(eps=1e-6, rot_frac=0.25)),
    "w1024_llama_d64": ("llama", 1024, 4, 64, 1e4, {}),
    "w1024_qwen35_d64_rot8": ("qwen3_5", 1024, 4, 64, 1e7, dict(eps=1e-6, rot_frac=0.125)),
}


def _case(name, layers):
    if name in CASES:
        return case(name, layers=layers)
    arch, h, hkv, d, theta, kw = WIDE[name]
    cfg = attn_config(arch, h, hkv, d, theta, layers=layers, **kw)
    return cfg, random_tensors(cfg, 0)


# P: 700 rows give fewer tiles than CUs for most cases (one tile per block); 20000 rows run every block
# over several tiles, with a ragged last tile row
@pytest.mark.parametrize("P", [700, 20000])
@pytest.mark.parametrize("name", sorted(CASES) + sorted(WIDE))
def test_batch_equals_per_layer(dev, name, P):
    from rfill import ops
    from rfill.model import FillModel
    nl = 3
    cfg, t = _case(name, nl)
    H, hkv, d = cfg["hidden_size"], cfg["num_key_value_heads"], cfg["head_dim"]
    layers = list(range(nl))
    m = FillModel(cfg, t, dev)
    b = inputs(P, H, seed=21).to(dev)
    W, B = _maps(H, layers, 22)
    W, B = [w.to(dev) for w in W], [c.to(dev) for c in B]
    pos = torch.arange(P, device=dev)
    cs = m.rope_table(pos)
    slot0, cap = 5, P + 5 + 64
    sentinel = -7.0
    ref_x, ref_s, ref_c = [], [], []
    for i in layers:
        x, s = ops.map_apply(b, W[i], B[i])
        w = m.W[i]
        kb = torch.full((hkv, cap, d), sentinel, dtype=torch.bfloat16, device=dev)
        vb = kb.clone()
        ops.norm_kv_write(x, s, m.eps, w["wkv"], hkv, d, w.get("k_norm"), m.knorm_kind, cs, kb, vb, slot0)
        ref_x.append(x)
        ref_s.append(s)
        ref_c.append((kb, vb))
    xs = [torch.empty(P, H, dtype=torch.bfloat16, device=dev) for _ in layers]
    ss = [torch.empty(P, H // 256, dtype=torch.float32, device=dev) for _ in layers]
    ops.map_apply_batch(b, W, B, xs, ss)
    kbs = [torch.full((hkv, cap, d), sentinel, dtype=torch.bfloat16, device=dev) for _ in layers]
    vbs = [k.clone() for k in kbs]
    ops.norm_kv_write_batch(xs, ss, m.eps, [m.W[i]["wkv"] for i in layers], hkv, d,
                            [m.W[i].get("k_norm") for i in layers], m.knorm_kind, cs, kbs, vbs, slot0)
    torch.cuda.synchronize()
    for i in layers:
        assert torch.equal(xs[i], ref_x[i]), f"layer {i}: x differs"
        assert torch.equal(ss[i], ref_s[i]), f"layer {i}: statistics differ"
        assert torch.equal(kbs[i], ref_c[i][0]), f"layer {i}: K differs"
        assert torch.equal(vbs[i], ref_c[i][1]), f"layer {i}: V differs"
        assert bool((kbs[i][:, :slot0] == sentinel).all()) and bool((kbs[i][:, slot0 + P:] == sentinel).all())
        assert bool((vbs[i][:, :slot0] == sentinel).all()) and bool((vbs[i][:, slot0 + P:] == sentinel).all())
    # layer 0's K / V against the oracle's fill of the same inputs (sampled rows at P = 20000)
    from oracle import model as OM
    sel = torch.arange(P) if P <= 1000 else torch.randperm(P, generator=torch.Generator().manual_seed(28))[:512].sort().values
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    om.fill(0, ref_x[0][sel.to(dev)].cpu(), sel, oc)
    ek = rel_err(kbs[0][:, (slot0 + sel).to(dev)], oc[0]["k"])
    ev = rel_err(vbs[0][:, (slot0 + sel).to(dev)], oc[0]["v"])
    print(f"{name} P {P}: K rel err {ek:.2e}, V rel err {ev:.2e} vs the oracle")
    assert ek < 1e-2 and ev < 1e-2


def test_batch_c2_shape(dev):
    """Four late layers at the Llama-8B 32K shape (P = 28672; 7168 map tiles and 3584 K / V tiles, 28 and
    14 per block): bitwise the per-layer unsplit launches; 256 sampled rows of one layer's K / V against
    the oracle's fill of those rows."""
    from oracle import model as OM
    from rfill import ops, synth
    from rfill.model import FillModel
    cfg = synth.LLAMA_8B
    layers = [16, 17, 18, 19]
    tensors = {}
    for i in layers:
        t, _, _ = synth.layer_weights(cfg, i, with_map=False)
        tensors.update(t)
    P, H = 28672, cfg["hidden_size"]
    m = FillModel(cfg, tensors, dev, layers=layers)
    b = synth.hidden_states(P, H).to(dev)
    W, B = _maps(H, layers, 23)
    W, B = [w.to(dev) for w in W], [c.to(dev) for c in B]
    pos = torch.arange(P, device=dev)
    cs = m.rope_table(pos)
    xs = [torch.empty(P, H, dtype=torch.bfloat16, device=dev) for _ in layers]
    ss = [torch.empty(P, H // 256, dtype=torch.float32, device=dev) for _ in layers]
    ops.map_apply_batch(b, W, B, xs, ss)
    kbs = [torch.zeros(8, P + 64, 128, dtype=torch.bfloat16, device=dev) for _ in layers]
    vbs = [k.clone() for k in kbs]
    ops.norm_kv_write_batch(xs, ss, m.eps, [m.W[i]["wkv"] for i in layers], 8, 128, [None] * 4, 0, cs, kbs, vbs, 0)
    for n, i in enumerate(layers):
        x, s = ops.map_apply(b, W[n], B[n])
        assert torch.equal(xs[n], x) and torch.equal(ss[n], s), f"layer {i}: map differs"
        kb, vb = torch.zeros_like(kbs[n]), torch.zeros_like(vbs[n])
        ops.norm_kv_write(x, s, m.eps, m.W[i]["wkv"], 8, 128, None, 0, cs, kb, vb, 0)
        assert torch.equal(kbs[n], kb) and torch.equal(vbs[n], vb), f"layer {i}: K / V differ"
        del x, s, kb, vb
    sel = torch.randperm(P, generator=torch.Generator().manual_seed(24))[:256].sort().values
    om = OM.OracleModel(cfg, tensors, dtype=torch.bfloat16, layers=layers)
    oc = om.new_cache()
    om.fill(17, xs[1][sel.to(dev)].cpu(), sel, oc)
    ek = rel_err(kbs[1][:, sel.to(dev)], oc[17]["k"])
    ev = rel_err(vbs[1][:, sel.to(dev)], oc[17]["v"])
    print(f"C2 batch layer 17: K rel err {ek:.2e}, V rel err {ev:.2e}")
    assert ek < 1e-2 and ev < 1e-2


def test_fill_late_groups_equal_per_layer(dev):
    """fill_late's grouped schedule (ATTN_GROUP attention layers per map launch and K / V launch) gives every
    layer the caches of per-layer unsplit launches, bitwise, with given exact-row inputs scattered in."""
    from rfill import ops
    from rfill.kva import ATTN_GROUP, Arm, Projector, fill_late
    from rfill.model import FillModel
    L, split, N, tail = 8, 2, 3000, 200
    cfg, t = case("qwen3_knorm", layers=L)
    H = cfg["hidden_size"]
    P = N - tail
    late = list(range(split, L))
    assert len(late) > ATTN_GROUP                      # at least one full group and a remainder
    Wl, Bl = _maps(H, late, 25)
    W, B = dict(zip(late, Wl)), dict(zip(late, Bl))
    h = inputs(N, H, seed=26).to(dev)
    rows = torch.tensor([3, 64, 65, 700, 2799])
    hr = inputs(5, H, seed=27)
    m = FillModel(cfg, t, dev)
    arm = Arm("ridgefill", split=split, tail=tail, fill="proj", projector=Projector(split, W, B))
    cache, got_p = fill_late(m, h, arm, exact_rows=rows, hr=hr.to(dev))
    torch.cuda.synchronize()
    assert got_p == P
    pos = torch.arange(P, device=dev)
    cs = m.rope_table(pos)
    for i in late:
        x, s = ops.map_apply(h[:P], W[i].to(dev), B[i].to(dev))
        ops.row_scatter(x, s, rows.to(dev), hr.to(dev))
        w = m.W[i]
        kb = torch.zeros(cfg["num_key_value_heads"], P + 64, cfg["head_dim"], dtype=torch.bfloat16, device=dev)
        vb = kb.clone()
        ops.norm_kv_write(x, s, m.eps, w["wkv"], m.n_kv, m.head_dim, w.get("k_norm"), m.knorm_kind, cs, kb, vb, 0)
        assert cache[i]["n"] == P
        assert torch.equal(cache[i]["k"], kb[:, :P]), f"layer {i}: K differs"
        assert torch.equal(cache[i]["v"], vb[:, :P]), f"layer {i}: V differs"


def test_fill_late_hybrid_groups_equal_per_layer(dev):
    """A hybrid late stack (GDN, GDN, GDN, attention, GDN, GDN) at width 1024 filled by fill_late's grouped
    schedule (one map launch per group, paired GDN fills with one in-projection launch, batched attention
    fills) against per-layer unsplit launches: every GDN conv and recurrent state and the attention layer's K
    / V bitwise equal."""
    from fill_cases import hybrid_config, hybrid_tensors
    from rfill import ops
    from rfill.kva import Arm, Projector, fill_late
    from rfill.model import FillModel
    kinds = ["gdn", "gdn", "gdn", "attn", "gdn", "gdn"]
    cfg = hybrid_config(kinds, hidden=1024)
    t = hybrid_tensors(cfg, seed=29)
    H, L, N, tail = cfg["hidden_size"], len(kinds), 2600, 100
    P = N - tail
    late = list(range(L))
    Wl, Bl = _maps(H, late, 30)
    W, B = dict(zip(late, Wl)), dict(zip(late, Bl))
    h = inputs(N, H, seed=31).to(dev)
    m = FillModel(cfg, t, dev)
    arm = Arm("ridgefill", split=0, tail=tail, fill="proj", projector=Projector(0, W, B))
    cache, _ = fill_late(m, h, arm)
    torch.cuda.synchronize()
    ref = m.new_cache()
    pos = torch.arange(P, device=dev)
    for i in late:
        x, s = ops.map_apply(h[:P], W[i].to(dev), B[i].to(dev))
        if kinds[i] == "attn":
            w = m.W[i]
            kb = torch.zeros(m.n_kv, P + 64, m.head_dim, dtype=torch.bfloat16, device=dev)
            vb = kb.clone()
            ops.norm_kv_write(x, s, m.eps, w["wkv"], m.n_kv, m.head_dim, w.get("k_norm"), m.knorm_kind,
                              m.rope_table(pos), kb, vb, 0)
            assert torch.equal(cache[i]["k"], kb[:, :P]) and torch.equal(cache[i]["v"], vb[:, :P]), f"layer {i}"
        else:
            m.fill(i, x, pos, ref, ssq=s)
            assert torch.equal(cache[i]["conv"], ref[i]["conv"]), f"layer {i}: conv state differs"
            assert torch.equal(cache[i]["rec"], ref[i]["rec"]), f"layer {i}: recurrent state differs"


def test_norm_linear_batch_ragged_entries(dev):
    """rf_norm_linear_batch with entries of different rows and widths in one launch (a GDN fill's two
    entries per layer: every row against the k | v | b | a rows, the last 3 rows against the q rows): each
    entry bitwise rf_norm_linear of it alone; the rows and columns outside the entries untouched."""
    from rfill import ops
    g = torch.Generator().manual_seed(21)
    P, H = 1000, 1024
    x = inputs(P, H, seed=22).to(dev)
    ssq = ops.row_ssq(x)
    w = [(torch.randn(n, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev) for n in (768, 256, 512)]
    out = torch.full((P, 1280), 3.0, dtype=torch.bfloat16, device=dev)
    ops.norm_linear_batch([x, x[P - 3:], x[:130]], [ssq, ssq[P - 3:], ssq[:130]], 1e-6, w,
                          [out[:, 512:], out[P - 3:, :256], out[:130, :512]])
    torch.cuda.synchronize()
    assert torch.equal(out[:, 512:], ops.norm_linear(x, ssq, 1e-6, w[0]))
    assert torch.equal(out[P - 3:, :256], ops.norm_linear(x[P - 3:], ssq[P - 3:], 1e-6, w[1]))
    assert torch.equal(out[:130, :512], ops.norm_linear(x[:130], ssq[:130], 1e-6, w[2]))
    assert bool((out[130:P - 3, :512] == 3.0).all()) and bool((out[P - 3:, 256:512] == 3.0).all())
