"""The allocation-free GDN fill (rf_gdn_fill_noalloc, the library's own device array as the workspace)
against rf_gdn_fill with a caller workspace, through the C ABI, bit for bit: two calls in a row on the same
GPU, the second with fewer rows (the array keeps the first call's contents), at the hybrid's widths
(16 key / 32 value heads: 39 chunks per pass, so the 9000-row call makes 4 passes); and the refusal of heads
whose one chunk exceeds the array."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _layer(dev, nk, nv, rows, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    C = 2 * nk * 128 + nv * 128
    pre = (0.5 * torch.randn(rows, C + 2 * nv, generator=g, device=dev)).to(torch.bfloat16)
    conv = (torch.rand(C, 4, generator=g, device=dev) - 0.5).to(torch.bfloat16)
    a_log = torch.log(16 * torch.rand(nv, generator=g, device=dev).clamp_min(1e-6))
    dt_bias = torch.ones(nv, device=dev)
    conv_in = (0.5 * torch.randn(3, C, generator=g, device=dev)).to(torch.bfloat16)
    state0 = 0.01 * torch.randn(nv, 128, 128, generator=g, device=dev)
    return pre, conv, a_log, dt_bias, conv_in, state0


def test_noalloc_gdn_fill_matches_the_workspace_entry_point(dev):
    from rfill import ops
    nk, nv = 16, 32
    for call, (rows, seed) in enumerate(((9000, 81), (700, 82))):       # the second call is smaller
        pre, conv, a_log, dt_bias, conv_in, state0 = _layer(dev, nk, nv, rows, seed)
        print(f"[no-alloc] call {call}: rows {rows}, heads {nk}/{nv}", flush=True)
        s_ref, s_got = state0.clone(), state0.clone()
        c_ref = ops.gdn_fill(pre, nk, nv, 128, 128, conv, conv_in, a_log, dt_bias, s_ref)
        c_got = ops.gdn_fill_noalloc(pre, nk, nv, 128, 128, conv, conv_in, a_log, dt_bias, s_got)
        torch.cuda.synchronize()
        assert torch.equal(s_got, s_ref) and torch.equal(c_got, c_ref)
        assert bool(torch.isfinite(s_got).all())


def test_noalloc_refuses_heads_beyond_the_array(dev):
    from rfill import ops
    nk = nv = 1024                                      # 61 MiB per chunk > 56 MiB
    C = 2 * nk * 128 + nv * 128
    pre = torch.zeros(1, C + 2 * nv, dtype=torch.bfloat16, device=dev)
    conv = torch.zeros(C, 4, dtype=torch.bfloat16, device=dev)
    st = torch.zeros(nv, 128, 128, device=dev)
    with pytest.raises(ValueError, match="scratch array"):
        ops.gdn_fill_noalloc(pre, nk, nv, 128, 128, conv, None, torch.zeros(nv, device=dev), torch.zeros(nv, device=dev), st)
