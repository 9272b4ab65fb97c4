"""Split K in the GEMM entry points (rf_map_apply, rf_norm_kv_write, rf_norm_q, rf_norm_linear with a
workspace of rf_gemm_workspace_bytes): for products with too few 256 x 256 tiles -- the exact rows'
and the tail's projections -- the K range is split over more blocks and the fp32 partials are added in
a fixed order before the same epilogue. Checked against a plain fp32 torch product and against the
unsplit kernel on the same inputs (bf16 bar 1e-2; split and unsplit differ only by fp32 summation order),
the same bits run to run, and nothing written past the rows."""
import pytest
import torch

from fill_cases import case, inputs, rel_err
from oracle import model as OM

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


@pytest.mark.parametrize("P,h_in,h_out", [(287, 4096, 4096), (300, 12288, 1024), (40, 2048, 512)])
def test_map_apply_split(dev, P, h_in, h_out):
    from rfill import ops
    g = torch.Generator().manual_seed(P)
    b = inputs(P, h_in, seed=P)
    w = (torch.randn(h_out, h_in, generator=g) / h_in ** 0.5).to(torch.bfloat16)
    c = (0.1 * torch.randn(h_out, generator=g)).to(torch.bfloat16)
    bd, wd, cd = b.to(dev), w.to(dev), c.to(dev)
    assert ops.gemm_workspace_bytes(P, h_out, h_in) > 0
    big = torch.full((P + 5, h_out), 7.0, dtype=torch.bfloat16, device=dev)
    xs, ss = ops.map_apply(bd, wd, cd, out=big[:P], workspace="auto")
    x2, s2 = ops.map_apply(bd, wd, cd, workspace="auto")
    xu, su = ops.map_apply(bd, wd, cd)
    torch.cuda.synchronize()
    ref = torch.nn.functional.linear(b.float(), w.float(), c.float())
    e_ref, e_un = rel_err(xs, ref), rel_err(xs, xu)
    print(f"map_apply {P}x{h_in}->{h_out}: split vs fp32 {e_ref:.2e}, split vs unsplit {e_un:.2e}, "
          f"unsplit vs fp32 {rel_err(xu, ref):.2e}")
    assert e_ref < TOL and e_un < TOL
    assert torch.equal(xs, x2) and torch.equal(ss, s2)
    assert bool((big[P:] == 7.0).all())
    assert torch.equal(ops.row_ssq(xs), ss)                          # the statistics of the rounded x


def test_norm_linear_and_norm_q_split(dev):
    """Row-scaled linear and the query projection (q_norm, RoPE at scattered positions) of 200 rows at
    hidden 2048 (2 and 4 tiles: K split 4 ways), split vs unsplit and vs the oracle's queries."""
    from fill_cases import attn_config, random_tensors
    from rfill import ops
    from rfill.model import FillModel
    cfg = attn_config("qwen3", 2048, 2, 128, 1e6, eps=1e-6)
    t = random_tensors(cfg, seed=5)
    H, R = cfg["hidden_size"], 200
    xc = inputs(R, H, seed=9)
    x = xc.to(dev)
    ssq = ops.row_ssq(x)
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(1024, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    assert ops.gemm_workspace_bytes(R, 1024, H) > 0
    a = ops.norm_linear(x, ssq, 1e-6, w, workspace="auto")
    u = ops.norm_linear(x, ssq, 1e-6, w)
    assert rel_err(a, u) < TOL
    m = FillModel(cfg, t, dev)
    wq = m._pack_rows(0)
    hq, d = m.n_heads, m.head_dim
    assert ops.gemm_workspace_bytes(R, hq * d, H) > 0
    pos = torch.randperm(3000, generator=g)[:R].sort().values
    cs = m.rope_table(torch.arange(3000, device=dev))
    q_s = ops.norm_q(x, ssq, m.eps, wq["wq"], hq, d, wq.get("q_norm"), m.knorm_kind, cs, pos.to(dev), workspace="auto")
    q_u = ops.norm_q(x, ssq, m.eps, wq["wq"], hq, d, wq.get("q_norm"), m.knorm_kind, cs, pos.to(dev))
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    want, _ = om.queries(0, om.in_norm(xc, om.W[0]["ln1"]), pos)          # [hq, R, d]
    want = want.transpose(0, 1).reshape(R, hq * d)
    e_su, e_o = rel_err(q_s, q_u), rel_err(q_s, want)
    print(f"norm_q split vs unsplit {e_su:.2e}, split vs oracle {e_o:.2e}; norm_linear split vs unsplit "
          f"{rel_err(a, u):.2e}")
    assert e_su < TOL and e_o < TOL


def test_norm_kv_write_split_matches_oracle(dev):
    """The tail's K / V write at a shape with too few tiles (few rows, one 256-column tile pair): split
    vs the oracle's fill and vs unsplit; slots exact."""
    from rfill import ops
    from rfill.model import FillModel
    cfg, t = case("qwen35_attn")                     # hidden 2048: K splits 4 ways; k_norm, partial RoPE
    P, H = 230, cfg["hidden_size"]
    x = inputs(P, H, seed=17)
    pos = torch.arange(P)
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    om.fill(0, x, pos, oc)
    m = FillModel(cfg, t, dev)
    w = m.W[0]
    xd = x.to(dev)
    ssq = ops.row_ssq(xd)
    cs = m.rope_table(pos.to(dev))
    N = w["wkv"].shape[0]
    assert ops.gemm_workspace_bytes(P, N, H) > 0
    kb = torch.full((m.n_kv, P + 70, m.head_dim), 5.0, dtype=torch.bfloat16, device=dev)
    vb = kb.clone()
    ku, vu = kb.clone(), vb.clone()
    ws = torch.empty(ops.gemm_workspace_bytes(P, N, H), dtype=torch.uint8, device=dev)
    kn = w.get("k_norm")
    ops.norm_kv_write(xd, ssq, m.eps, w["wkv"], m.n_kv, m.head_dim, kn, m.knorm_kind, cs, kb, vb, 3, workspace=ws)
    ops.norm_kv_write(xd, ssq, m.eps, w["wkv"], m.n_kv, m.head_dim, kn, m.knorm_kind, cs, ku, vu, 3)
    torch.cuda.synchronize()
    ek, ev = rel_err(kb[:, 3:3 + P], oc[0]["k"]), rel_err(vb[:, 3:3 + P], oc[0]["v"])
    print(f"norm_kv_write split: K {ek:.2e} V {ev:.2e} vs oracle; vs unsplit K {rel_err(kb, ku):.2e}")
    assert ek < TOL and ev < TOL and rel_err(kb, ku) < TOL
    assert bool((kb[:, :3] == 5.0).all() and (kb[:, 3 + P:] == 5.0).all() and (vb[:, 3 + P:] == 5.0).all())


def test_last_wave_split(dev):
    """A product whose last wave of tile rows is at most half full (10240 rows x 2048: 40 tile rows of
    8 tiles, 32 per wave) runs rows [0, 8192) fused and rows [8192, 10240) split in K: map apply and
    the fused norm + K / V + RoPE write against their unsplit runs and the oracle, the rows' statistics
    bitwise those of the rounded x, the cache slots exact."""
    from fill_cases import attn_config, random_tensors
    from rfill import ops
    from rfill.model import FillModel
    P, H = 10240, 2048
    assert ops.gemm_workspace_bytes(P, 2048, H) == 4 * 2048 * 2048 * 4       # 4 splits of the last 2048 rows
    g = torch.Generator().manual_seed(7)
    b = inputs(P, H, seed=8).to(dev)
    w = (torch.eye(H) + 0.02 * torch.randn(H, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    c = (1e-3 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    xs, ss = ops.map_apply(b, w, c, workspace="auto")
    xu, su = ops.map_apply(b, w, c)
    torch.cuda.synchronize()
    assert torch.equal(xs[:8192], xu[:8192]) and torch.equal(ss[:8192], su[:8192])     # the fused rows
    assert rel_err(xs, xu) < TOL and torch.equal(ops.row_ssq(xs), ss)
    cfg = attn_config("llama", H, 8, 128, 5e5)                  # K and V: 2 x 8 heads x 128 = 2048 columns
    t = random_tensors(cfg, seed=9)
    m = FillModel(cfg, t, dev)
    x = xu.cpu()
    pos = torch.arange(P)
    c0 = m.new_cache()
    m.fill(0, xu, pos.to(dev), c0)                               # FillModel.fill passes the workspace
    wk = m.W[0]
    kb = torch.empty(8, P + 64, 128, dtype=torch.bfloat16, device=dev)
    vb = torch.empty_like(kb)
    ops.norm_kv_write(xu, su, m.eps, wk["wkv"], 8, 128, None, 0, m.rope_table(pos.to(dev)), kb, vb, 0)
    torch.cuda.synchronize()
    om = OM.OracleModel(cfg, t, dtype=torch.bfloat16)
    oc = om.new_cache()
    om.fill(0, x, pos, oc)
    ek, ev = rel_err(c0[0]["k"], oc[0]["k"]), rel_err(c0[0]["v"], oc[0]["v"])
    ek_tail = rel_err(c0[0]["k"][:, 8192:], oc[0]["k"][:, 8192:])
    print(f"last-wave split: map x vs unsplit {rel_err(xs, xu):.2e}; K {ek:.2e} V {ev:.2e} (split rows K {ek_tail:.2e}) "
          f"vs oracle; vs unsplit K {rel_err(c0[0]['k'], kb[:, :P]):.2e}")
    assert ek < TOL and ev < TOL and ek_tail < TOL
    assert torch.equal(c0[0]["k"][:, :8192], kb[:, :8192])      # the fused rows: the same kernel, the same bits
    assert rel_err(c0[0]["k"], kb[:, :P]) < TOL and rel_err(c0[0]["v"], vb[:, :P]) < TOL
    assert c0[0]["n"] == P


@pytest.mark.parametrize("P", [1, 3, 33, 129, 160, 161, 287, 512])
def test_few_rows_products(dev, P):
    """Products of at most 512 rows (k_rows_partial: every row of a row block against 128 weight rows). At
    hidden 512 the K range is one split, and the row-scaled linear is bit-identical to the unsplit kernel
    (the same MFMA, operands and K order); at hidden 4096 (split 2 .. 8 ways) it agrees with the unsplit
    kernel and a plain fp32 product, and nothing is written past the rows."""
    from rfill import ops
    g = torch.Generator().manual_seed(100 + P)
    for H, N in ((512, 1024), (4096, 2048)):
        xc = inputs(P, H, seed=P + H)
        x = xc.to(dev)
        ssq = ops.row_ssq(x)
        w = (torch.randn(N, H, generator=g) / H ** 0.5).to(torch.bfloat16)
        wd = w.to(dev)
        nbytes = ops.gemm_workspace_bytes(P, N, H)
        assert nbytes % (P * N * 4) == 0 and (nbytes == P * N * 4 if H == 512 else nbytes >= 2 * P * N * 4)
        big = torch.full((P + 3, N), 7.0, dtype=torch.bfloat16, device=dev)
        a = ops.norm_linear(x, ssq, 1e-6, wd, out=big[:P], workspace="auto")
        u = ops.norm_linear(x, ssq, 1e-6, wd)
        torch.cuda.synchronize()
        xn = xc.float() * torch.rsqrt(xc.float().pow(2).mean(1, keepdim=True) + 1e-6)
        ref = xn @ w.float().t()
        print(f"P {P} H {H}: rows-kernel vs unsplit {rel_err(a, u):.2e}, vs fp32 {rel_err(a, ref):.2e}")
        if H == 512:
            assert torch.equal(a, u)
        assert rel_err(a, u) < TOL and rel_err(a, ref) < TOL
        assert bool((big[P:] == 7.0).all())
