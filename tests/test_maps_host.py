"""Map formats on the host: the oracle's i8_row128 expansion (code/c5/convert.py:91-109) pinned against an
independent computation (float64 products, round-to-nearest-even to bf16 by integer arithmetic on the
bit pattern), hand-worked values including a tie, the engine -> fill layout of the GDN terminal-state
correction (code/c5/convert.py:7-8 vs code/kva/ops.py:4-6), and the loader's refusals (no GPU)."""
import numpy as np
import pytest
import torch

from oracle import kva as okva


def rne_bf16(x64):
    """float64 values (exactly representable in fp32) -> bf16 bit patterns, round to nearest even."""
    u = np.asarray(x64, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def bf16_bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def test_dequant_known_values():
    codes = torch.zeros(1, 128, dtype=torch.int8)
    codes[0, :4] = torch.tensor([1, -2, 127, -128], dtype=torch.int8)
    m = okva.dequant_i8_row128(codes, torch.tensor([[0.5]], dtype=torch.bfloat16), torch.tensor([0.25], dtype=torch.bfloat16))
    assert m.shape == (1, 129)
    assert m[0, :4].tolist() == [0.5, -1.0, 63.5, -64.0] and m[0, -1].item() == 0.25
    # 127 * (1 + 2^-7) = 127.9921875 rounds up to 128 in bf16; 3 * bf16(1/3) = 1.001953125 rounds down to 1
    s = torch.tensor([[1.0078125]], dtype=torch.bfloat16)
    codes[0, 0] = 127
    assert okva.dequant_i8_row128(codes, s, torch.zeros(1, dtype=torch.bfloat16)).to(torch.bfloat16)[0, 0].item() == 128.0
    codes[0, 0] = 3
    s3 = torch.tensor([[1 / 3]], dtype=torch.bfloat16)
    assert s3.item() == 0.333984375
    assert okva.dequant_i8_row128(codes, s3, torch.zeros(1, dtype=torch.bfloat16)).to(torch.bfloat16)[0, 0].item() == 1.0


def test_dequant_ties_round_to_even():
    # 3 * 1.0078125 = 3.0234375 (fp32 0x40418000) and 3 * 1.0234375 = 3.0703125 (0x40448000) lie exactly
    # halfway between two bf16 values: the first rounds up to 0x4042, the second down to 0x4044
    codes = torch.zeros(1, 256, dtype=torch.int8)
    codes[0, 0], codes[0, 128] = 3, 3
    s = torch.tensor([[1.0078125, 1.0234375]], dtype=torch.bfloat16)
    got = okva.dequant_i8_row128(codes, s, torch.zeros(1, dtype=torch.bfloat16)).to(torch.bfloat16)
    bits = bf16_bits(got[0, [0, 128]].contiguous())
    assert [int(np.float32(v).view(np.uint32)) & 0xFFFF for v in (3.0234375, 3.0703125)] == [0x8000, 0x8000]
    assert bits.tolist() == [0x4042, 0x4044]
    assert bits.tolist() == rne_bf16([3.0234375, 3.0703125]).tolist()


def test_dequant_matches_independent_rounding():
    g = torch.Generator().manual_seed(3)
    rows, width = 37, 512
    codes = torch.randint(-128, 128, (rows, width), generator=g, dtype=torch.int16).to(torch.int8)
    scale = (torch.rand(rows, width // 128, generator=g) * 0.02 + 1e-4).to(torch.bfloat16)
    bias = torch.randn(rows, generator=g).to(torch.bfloat16)
    m = okva.dequant_i8_row128(codes, scale, bias).to(torch.bfloat16)
    prod = codes.numpy().astype(np.float64) * np.repeat(scale.float().numpy().astype(np.float64), 128, axis=1)
    assert np.array_equal(bf16_bits(m[:, :width].contiguous()), rne_bf16(prod))
    assert torch.equal(m[:, -1], bias)


def test_projector_from_i8_row128_splits_weight_and_bias():
    g = torch.Generator().manual_seed(4)
    t = {}
    for L in (5, 6):
        t[f"proj.{L}.codes"] = torch.randint(-128, 128, (64, 256), generator=g, dtype=torch.int16).to(torch.int8)
        t[f"proj.{L}.scale"] = (torch.rand(64, 2, generator=g) * 0.01).to(torch.bfloat16)
        t[f"proj.{L}.bias"] = torch.randn(64, generator=g).to(torch.bfloat16)
    p = okva.projector_i8_row128(t, 5)
    assert sorted(p.W) == [5, 6] and p.W[5].shape == (64, 256) and p.b[6].shape == (64,)
    full = okva.dequant_i8_row128(t["proj.6.codes"], t["proj.6.scale"], t["proj.6.bias"]).to(torch.bfloat16)
    assert torch.equal(p.W[6], full[:, :-1]) and torch.equal(p.b[6], t["proj.6.bias"])


def test_st_from_engine_transposes():
    from rfill.kva import st_from_engine
    eng = torch.arange(2 * 3 * 4, dtype=torch.float32).view(2, 3, 4)      # [heads, V, K]
    out = st_from_engine({"27": eng})
    assert list(out) == [27] and out[27].shape == (2, 4, 3)
    assert out[27][1, 2, 0].item() == eng[1, 0, 2].item()                 # [h, k, v] = engine [h, v, k]
    with pytest.raises(ValueError):
        st_from_engine({1: eng[0]})


def test_load_i8_row128_refuses_bad_tensors():
    from rfill.kva import load_i8_row128
    ok = {"proj.5.codes": torch.zeros(8, 256, dtype=torch.int8), "proj.5.scale": torch.zeros(8, 2, dtype=torch.bfloat16),
          "proj.5.bias": torch.zeros(8, dtype=torch.bfloat16)}
    with pytest.raises(ValueError):
        load_i8_row128({}, 5)
    bad = dict(ok); del bad["proj.5.bias"]
    with pytest.raises(ValueError):
        load_i8_row128(bad, 5)
    bad = dict(ok, **{"proj.5.scale": torch.zeros(8, 3, dtype=torch.bfloat16)})
    with pytest.raises(ValueError):
        load_i8_row128(bad, 5)
    bad = dict(ok, **{"proj.5.codes": torch.zeros(8, 256, dtype=torch.int16)})
    with pytest.raises(ValueError):
        load_i8_row128(bad, 5)
