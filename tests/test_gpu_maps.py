"""The i8_row128 map layout on the device: rf_dequant_i8_rows against the oracle's expansion
(code/c5/convert.py:91-109) bit for bit, at the release's map shape [2560, 10240] and at small, strided
and other-group cases; load_i8_row128's Projector against the oracle's, maps bitwise and its map apply
within the bf16 bar; the kernel's refusals."""
import pytest
import torch

from oracle import kva as okva

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def release_like(rows, width, seed, group=128):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(-128, 128, (rows, width), generator=g, dtype=torch.int16).to(torch.int8)
    scale = (torch.rand(rows, width // group, generator=g) * 2e-3 + 1e-5).to(torch.bfloat16)
    return codes, scale


@pytest.mark.parametrize("rows,width", [(2560, 10240), (3, 256), (130, 384)])
def test_dequant_matches_oracle_bitwise(dev, rows, width):
    from rfill import ops
    codes, scale = release_like(rows, width, rows)
    want = okva.dequant_i8_row128(codes, scale, torch.zeros(rows, dtype=torch.bfloat16))[:, :width].to(torch.bfloat16)
    got = ops.dequant_i8_rows(codes.to(dev), scale.to(dev), 128)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want), (rows, width)
    print(f"dequant {rows} x {width}: bit-identical to the reference's expansion")


def test_dequant_strided_and_group_32(dev):
    from rfill import ops
    codes, scale = release_like(64, 512, 7, group=32)
    big = torch.zeros(64, 640, dtype=torch.int8)
    big[:, :512] = codes
    out = torch.zeros(64, 528, dtype=torch.bfloat16, device=dev)
    ops.dequant_i8_rows(big.to(dev)[:, :512], scale.to(dev), 32, out=out[:, :512])
    torch.cuda.synchronize()
    want = (codes.float() * scale.float().repeat_interleave(32, 1)).to(torch.bfloat16)
    assert torch.equal(out[:, :512].cpu(), want)
    assert not bool(out[:, 512:].any()), "nothing written past the row width"


def test_loader_matches_oracle_projector(dev):
    from rfill.kva import load_i8_row128
    g = torch.Generator().manual_seed(9)
    t = {}
    for L in (16, 17):
        c, s = release_like(512, 1024, L)
        t[f"proj.{L}.codes"], t[f"proj.{L}.scale"] = c, s
        t[f"proj.{L}.bias"] = (1e-2 * torch.randn(512, generator=g)).to(torch.bfloat16)
    p = load_i8_row128(t, 16, device=dev)
    o = okva.projector_i8_row128(t, 16)
    for L in (16, 17):
        assert torch.equal(p.W[L].cpu(), o.W[L]) and torch.equal(p.b[L].cpu(), o.b[L])
    b = torch.randn(300, 1024, generator=g).to(torch.bfloat16)
    x = p(17, b.to(dev)).float().cpu()
    ref = o(17, b.float()).float()
    err = ((x - ref).norm() / ref.norm()).item()
    print(f"map apply with the loaded i8_row128 map: rel err vs the oracle {err:.2e}")
    assert err < 1e-2


def test_dequant_refuses(dev):
    from rfill import ops
    codes, scale = release_like(4, 256, 1)
    with pytest.raises(ValueError):
        ops.dequant_i8_rows(codes.to(dev), scale.to(dev), 100)        # group does not divide the width
    with pytest.raises(ValueError):
        ops.dequant_i8_rows(codes.to(dev), scale[:, :1].to(dev), 128)
    c8, s8 = release_like(4, 256, 2, group=8)
    with pytest.raises(ValueError, match="group"):                     # refused by the C ABI: group % 16
        ops.dequant_i8_rows(c8.to(dev), s8.to(dev), 8)
