"""The GGUF container reader (rfill.gguf) on hand-assembled bytes, and the oracle's ggml dequantisation
(oracle.kva.dequant_gguf) pinned by hand-worked values and an independent float64 computation with a
round-to-nearest-even on the bf16 bit patterns."""
import struct

import numpy as np
import pytest
import torch

import gguf_writer
from oracle import kva as okva
from test_maps_host import bf16_bits, rne_bf16


def test_reader_on_hand_assembled_bytes(tmp_path):
    """One string and one u32 entry, one F32 [ne 8, 2] tensor: every field laid out by hand from the spec."""
    vals = np.arange(16, dtype=np.float32) - 3.5
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 2)
    head += struct.pack("<Q", 4) + b"k.ab" + struct.pack("<IQ", 8, 3) + b"xyz"
    head += struct.pack("<Q", 3) + b"k.n" + struct.pack("<II", 4, 77)
    head += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2) + struct.pack("<QQ", 8, 2) + struct.pack("<IQ", 0, 0)
    pad = (-len(head)) % 32
    path = tmp_path / "a.gguf"
    path.write_bytes(head + b"\0" * pad + vals.tobytes())
    from rfill import gguf
    meta, ts = gguf.read(path)
    assert meta == {"k.ab": "xyz", "k.n": 77}
    t = ts["t"]
    assert t.ne == (8, 2) and t.shape == (2, 8) and t.ggml_type == 0 and t.data.shape == (2, 32)
    assert np.array_equal(np.array(t.data).view(np.float32), vals.reshape(2, 8))
    # the test writer lays files out the same way
    gguf_writer.write(tmp_path / "b.gguf", [("k.ab", "str", "xyz"), ("k.n", "u32", 77)],
                      [("t", (8, 2), 0, vals.tobytes())])
    assert (tmp_path / "b.gguf").read_bytes() == path.read_bytes()


def test_reader_refuses(tmp_path):
    from rfill import gguf
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + b"\0" * 40)
    with pytest.raises(gguf.GGUFError, match="not a GGUF"):
        gguf.read(p)
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    with pytest.raises(gguf.GGUFError, match="version 1"):
        gguf.read(p)
    gguf_writer.write(p, [], [("q4", (32, 1), 2, b"\0" * 18)])        # Q4_0: not a map type
    with pytest.raises(gguf.GGUFError, match="ggml type 2"):
        gguf.read(p)
    gguf_writer.write(p, [], [("t", (8, 2), 0, b"\0" * 64)])
    p.write_bytes(p.read_bytes()[:-8])
    with pytest.raises(gguf.GGUFError, match="outside the file"):
        gguf.read(p)


def test_q8_0_known_values():
    blk = np.zeros((1, 34), dtype=np.uint8)
    blk[0, :2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    blk[0, 2:6] = np.array([1, -2, 127, -128], dtype=np.int8).view(np.uint8)
    v = okva.dequant_gguf(blk, 8, 32)
    assert v.shape == (1, 32) and v[0, :5].tolist() == [0.5, -1.0, 63.5, -64.0, 0.0]
    # fp16(1/3) = 0.333251953125; times 3 = 0.999755859375, which rounds to 1.0 in bf16; times 127 =
    # 42.322998046875, between bf16 42.25 and 42.5, nearer 42.25
    blk[0, :2] = np.array([1 / 3], dtype=np.float16).view(np.uint8)
    blk[0, 2:4] = np.array([3, 127], dtype=np.int8).view(np.uint8)
    v = okva.dequant_gguf(blk, 8, 32)
    assert v[0, 0].item() == 0.999755859375 and v[0, 1].item() == 42.322998046875
    assert v[0, :2].to(torch.bfloat16).float().tolist() == [1.0, 42.25]


def test_dequant_against_float64():
    rng = np.random.default_rng(0)
    raw = gguf_writer.q8_0(7, 96, rng)
    d = raw.reshape(7, 3, 34)[:, :, :2].copy().view(np.float16).astype(np.float64)
    q = raw.reshape(7, 3, 34)[:, :, 2:].copy().view(np.int8).astype(np.float64)
    want = (d * q).reshape(7, 96)
    v = okva.dequant_gguf(raw, 8, 96)
    assert np.array_equal(v.double().numpy(), want)
    assert np.array_equal(bf16_bits(v.to(torch.bfloat16)), rne_bf16(want))
    # F16, including subnormals and the largest finite value
    h = rng.standard_normal((5, 64)).astype(np.float16)
    h[0, :4] = np.array([6.1e-5, 3e-7, -65504.0, 0.0], dtype=np.float16)
    v = okva.dequant_gguf(h.view(np.uint8), 1, 64)
    assert np.array_equal(v.double().numpy(), h.astype(np.float64))
    assert np.array_equal(bf16_bits(v.to(torch.bfloat16)), rne_bf16(h.astype(np.float64)))
    # BF16 widens exactly; F32 as stored
    b = rne_bf16(rng.standard_normal((2, 16)))
    assert np.array_equal(bf16_bits(okva.dequant_gguf(b.view(np.uint8), 30, 16).to(torch.bfloat16)), b)
    f = rng.standard_normal((2, 16)).astype(np.float32)
    assert np.array_equal(okva.dequant_gguf(f.view(np.uint8), 0, 16).numpy(), f)
