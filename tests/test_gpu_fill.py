"""GPU parity of the attention-layer fill (rf_map_apply, rf_row_ssq, rf_row_scatter, rf_rope_table,
rf_norm_kv_write, rf_rope_kv_write) against the CPU oracle on identical seeded inputs.

Bars: cache slot and row placement bit-exact; copies (scatter, V passthrough) bit-exact; filled K / V
within relative Frobenius error 1e-2 of the oracle (bf16 path); RoPE arithmetic bit-exact given the
same cos / sin table; results bitwise reproducible run to run."""
import pytest
import torch

from fill_cases import CASES, case, inputs, rel_err
from oracle import model as OM
from oracle import ops as oops

pytestmark = pytest.mark.gpu
KV_TOL = 1e-2          # relative Frobenius bound for bf16 fill outputs


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _oracle_fill(cfg, tensors, x, pos, i=0):
    m = OM.OracleModel(cfg, tensors, dtype=torch.bfloat16)
    c = m.new_cache()
    m.fill(i, x, pos, c)
    return c[i]


def test_map_apply_matches_linear(dev):
    from rfill import ops
    g = torch.Generator().manual_seed(0)
    P, h_in, h_out = 1000, 512, 768
    b = inputs(P, h_in, seed=3)
    w = (torch.randn(h_out, h_in, generator=g) / h_in ** 0.5).to(torch.bfloat16)
    c = (0.1 * torch.randn(h_out, generator=g)).to(torch.bfloat16)
    big = torch.full((P + 7, h_out), 7.0, dtype=torch.bfloat16, device=dev)
    x, ssq = ops.map_apply(b.to(dev), w.to(dev), c.to(dev), out=big[:P])
    torch.cuda.synchronize()
    ref = torch.nn.functional.linear(b, w, c)
    err = rel_err(x, ref)
    print(f"map_apply rel err {err:.2e}, identical {float((x.cpu() == ref).float().mean()):.4f}")
    assert err < KV_TOL
    assert bool((big[P:] == 7.0).all()), "rows past P were written"
    xf = x.float().cpu()
    want = (xf * xf).view(P, h_out // 256, 256).sum(-1)
    assert rel_err(ssq, want) < 1e-6


def test_row_ssq_equals_map_apply_partials_bitwise(dev):
    from rfill import ops
    P, h = 777, 1024
    b = inputs(P, 512, seed=4).to(dev)
    w = (torch.randn(h, 512, generator=torch.Generator().manual_seed(1)) / 512 ** 0.5).to(torch.bfloat16).to(dev)
    x, ssq = ops.map_apply(b, w, None)
    assert torch.equal(ops.row_ssq(x), ssq)


def test_row_scatter_is_bit_exact(dev):
    from rfill import ops
    P, h = 900, 512
    x = inputs(P, h, seed=5).to(dev)
    before = x.clone()
    ssq = ops.row_ssq(x)
    rows = torch.tensor([0, 3, 4, 100, 511, 899], device=dev)
    hr = inputs(6, h, seed=6).to(dev)
    ops.row_scatter(x, ssq, rows, hr)
    ref = before.index_copy(0, rows, hr)
    assert torch.equal(x, ref)
    assert torch.equal(ssq, ops.row_ssq(ref))


@pytest.mark.parametrize("name", sorted(CASES))
def test_fill_matches_oracle(dev, name):
    from rfill.model import FillModel
    cfg, t = case(name)
    P = 1792
    x = inputs(P, cfg["hidden_size"], seed=7)
    pos = torch.arange(P)
    ref = _oracle_fill(cfg, t, x, pos)
    m = FillModel(cfg, t, dev)
    cache = m.new_cache()
    m.fill(0, x.to(dev), pos.to(dev), cache)
    torch.cuda.synchronize()
    c = cache[0]
    assert c["n"] == P and c["kbuf"].shape[1] == P + 64
    ek, ev = rel_err(c["k"], ref["k"]), rel_err(c["v"], ref["v"])
    print(f"{name}: K rel err {ek:.2e}, V rel err {ev:.2e}")
    assert ek < KV_TOL and ev < KV_TOL


def test_fill_is_deterministic_and_appends(dev):
    """Two runs give the same bits; a fill of P1 rows then P2 rows equals one fill of P1 + P2 rows,
    bitwise (rows are independent), with the second call's rows at slots P1.. (slot = append order)."""
    from rfill.model import FillModel
    cfg, t = case("qwen3_knorm")
    x = inputs(1300, cfg["hidden_size"], seed=8).to(dev)
    pos = torch.arange(1300, device=dev)
    m = FillModel(cfg, t, dev)
    one, two, again = m.new_cache(), m.new_cache(), m.new_cache()
    m.fill(0, x, pos, one)
    m.fill(0, x, pos, again)
    m.fill(0, x[:1000], pos[:1000], two)
    m.fill(0, x[1000:], pos[1000:], two)                 # grows the buffer: old rows copied
    assert torch.equal(one[0]["k"], again[0]["k"]) and torch.equal(one[0]["v"], again[0]["v"])
    assert two[0]["n"] == 1300 and two[0]["kbuf"].shape[1] == 1300 + 64
    assert torch.equal(one[0]["k"], two[0]["k"]) and torch.equal(one[0]["v"], two[0]["v"])


def test_rope_table_matches_reference_tables(dev):
    """The device table equals bf16(cos / sin(float(pos) * inv_freq)) up to rare 1-ulp differences of
    the fp32 cos / sin before rounding (positions up to 131071)."""
    from rfill import ops
    inv = ops.inv_freq_default(5e5, 128)
    pos = torch.cat((torch.arange(4096), torch.randint(0, 131072, (4096,), generator=torch.Generator().manual_seed(2))))
    cs = ops.rope_table(pos.to(dev), inv.to(dev)).cpu()
    cos, sin = oops.rope_cos_sin(oops.inv_freq_default(5e5, 128), pos, torch.bfloat16)
    ref = torch.cat((cos[:, :64], sin[:, :64]), 1)
    same = (cs == ref).float().mean().item()
    ulp = (cs.view(torch.int16).int() - ref.view(torch.int16).int()).abs().max().item()
    print(f"rope table identical fraction {same:.6f}, max ulp {ulp}")
    assert same > 0.999 and ulp <= 1
    assert torch.equal(ops.inv_freq_default(5e5, 128), oops.inv_freq_default(5e5, 128))
    l3 = (500000.0, 128, 8.0, 1.0, 4.0, 8192)
    assert torch.equal(ops.inv_freq_llama3(*l3), oops.inv_freq_llama3(*l3))


@pytest.mark.parametrize("name", ["llama_c1", "qwen35_attn"])
def test_fill_kv_rope_bitwise_given_table(dev, name):
    """fill_kv from given pre-RoPE K / V: with the device's own cos / sin table fed to the oracle's
    apply_rope, K is bitwise the oracle's, V a bitwise copy, slots in append order."""
    from rfill.model import FillModel
    cfg, t = case(name)
    hkv, d = cfg["num_key_value_heads"], cfg["head_dim"]
    m = FillModel(cfg, t, dev)
    P = 700
    g = torch.Generator().manual_seed(11)
    k = torch.randn(P, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(P, hkv, d, generator=g).to(torch.bfloat16)
    pos = torch.arange(100, 100 + P)
    cache = m.new_cache()
    m.fill_kv(0, k.to(dev), v.to(dev), pos.to(dev), cache)
    cs = m.rope_table(pos.to(dev)).cpu()
    half = m.rot // 2
    cos = torch.cat((cs[:, :half], cs[:, :half]), 1)
    sin = torch.cat((cs[:, half:], cs[:, half:]), 1)
    ref_k = oops.apply_rope(k.transpose(0, 1), cos, sin)
    assert torch.equal(cache[0]["k"].cpu(), ref_k)
    assert torch.equal(cache[0]["v"].cpu(), v.transpose(0, 1))


def test_fill_full_c2_layer_rows(dev):
    """One late layer at the Llama-8B 32K shape (P = 28672 rows): 384 random rows against the oracle on
    just those rows (fill is row-independent), every slot < P written, slots >= P untouched."""
    from rfill import synth
    from rfill.model import FillModel
    cfg = synth.LLAMA_8B
    t, _, _ = synth.layer_weights(cfg, 16, with_map=False)
    P = 28672
    x = synth.hidden_states(P, cfg["hidden_size"])
    m = FillModel(cfg, t, dev, layers=[16])
    cache = m.new_cache()
    cap = P + 64
    sentinel = torch.full((8, cap, 128), -3.0, dtype=torch.bfloat16, device=dev)
    cache[16] = dict(kbuf=sentinel.clone(), vbuf=sentinel.clone(), n=0)
    m.fill(16, x.to(dev), torch.arange(P, device=dev), cache)
    torch.cuda.synchronize()
    k, v = cache[16]["kbuf"], cache[16]["vbuf"]
    assert bool((k[:, P:] == -3.0).all()) and bool((v[:, P:] == -3.0).all())
    assert bool(torch.isfinite(k[:, :P].float()).all()) and bool(torch.isfinite(v[:, :P].float()).all())
    sel = torch.randperm(P, generator=torch.Generator().manual_seed(5))[:384].sort().values
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16, layers=[16])
    oc = om.new_cache()
    om.fill(16, x[sel], sel, oc)
    ek = rel_err(k[:, sel.to(dev)], oc[16]["k"])
    ev = rel_err(v[:, sel.to(dev)], oc[16]["v"])
    print(f"C2 layer: K rel err {ek:.2e}, V rel err {ev:.2e}")
    assert ek < KV_TOL and ev < KV_TOL


def test_fill_late_proj_with_exact_rows(dev):
    """finish()'s fill loop on a C1-shaped model (3 late layers): projector maps, then the exact rows'
    inputs scattered in, then the fill; every late layer's cache against the oracle's same steps."""
    from rfill.kva import Arm, Projector, fill_late
    from rfill.model import FillModel
    cfg, t = case("llama_c1", layers=8)
    N, tail, split = 2048, 256, 5
    P = N - tail
    h = inputs(N, cfg["hidden_size"], seed=12)
    g = torch.Generator().manual_seed(13)
    H = cfg["hidden_size"]
    W = {i: (torch.eye(H) + 0.05 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16)
         for i in range(split, 8)}
    B = {i: (1e-2 * torch.randn(H, generator=g)).to(torch.bfloat16) for i in range(split, 8)}
    rows = torch.randperm(P, generator=g)[:18].sort().values
    hr = inputs(18, H, seed=14)
    arm = Arm("ridgefill", split=split, tail=tail, fill="proj", projector=Projector(split, W, B))
    m = FillModel(cfg, t, dev)
    cache, P_got = fill_late(m, h.to(dev), arm, exact_rows=rows, hr=hr.to(dev))
    assert P_got == P
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    pos = torch.arange(P)
    for i in range(split, 8):
        x = torch.nn.functional.linear(h[:P], W[i], B[i]).index_copy(0, rows, hr)
        om.fill(i, x, pos, oc)
        ek, ev = rel_err(cache[i]["k"], oc[i]["k"]), rel_err(cache[i]["v"], oc[i]["v"])
        er = rel_err(cache[i]["k"][:, rows.to(dev)], oc[i]["k"][:, rows])
        print(f"layer {i}: K {ek:.2e} V {ev:.2e} exact-row K {er:.2e}")
        assert ek < KV_TOL and ev < KV_TOL and er < KV_TOL
        assert cache[i]["n"] == P


def test_bad_inputs_raise_before_launch(dev):
    from rfill import ops
    from rfill._lib import UnsupportedArchitecture
    from rfill.kva import check_rows
    x = torch.zeros(10, 200, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.row_ssq(x)                                           # H not a multiple of 256
    with pytest.raises(ValueError):
        check_rows([3, 3, 5], 10)
    with pytest.raises(ValueError):
        check_rows([1, 12], 10)
    kb = torch.zeros(2, 20, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):                              # rows past the buffer's capacity
        ops.rope_kv_write(torch.zeros(30, 2, 64, dtype=torch.bfloat16, device=dev),
                          torch.zeros(30, 2, 64, dtype=torch.bfloat16, device=dev),
                          torch.zeros(30, 64, dtype=torch.bfloat16, device=dev), kb, kb.clone(), 0)
    with pytest.raises(UnsupportedArchitecture):                 # rot / 2 = 6: not a supported rotation
        ops.rope_kv_write(torch.zeros(4, 2, 64, dtype=torch.bfloat16, device=dev),
                          torch.zeros(4, 2, 64, dtype=torch.bfloat16, device=dev),
                          torch.zeros(4, 12, dtype=torch.bfloat16, device=dev), kb, kb.clone(), 0)


def test_mfma_ceiling_probe_runs(dev):
    """rf_mfma_ceiling (bench.py's power-ceiling measurement): every thread stores a finite sum; a short
    output buffer is refused before any launch."""
    from rfill import ops
    out = torch.full((4 * 256,), float("nan"), device=dev)
    ops.mfma_ceiling(4, 10, out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool((out != 0).any())
    with pytest.raises(ValueError, match="needs"):
        ops.mfma_ceiling(8, 10, out)
