"""GPU parity of the GGUF map loader: rf_dequant_gguf_rows bit-identical to the oracle's ggml
dequantisation cast to bf16 (round to nearest even) for F32, F16, Q8_0 and BF16, and load_gguf on an
adapter file (Q8_0 and F16 maps, F32 biases, a linear-attention layer with its state correction)."""
import numpy as np
import pytest
import torch

import gguf_writer
from oracle import kva as okva

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from rfill import _lib
    _lib.load()
    return torch.device("cuda")


def _raw(gt, rows, width, rng):
    if gt == 8:
        return gguf_writer.q8_0(rows, width, rng)
    x = rng.standard_normal((rows, width)) * 0.05
    if gt == 0:
        return x.astype(np.float32).view(np.uint8)
    if gt == 1:
        return x.astype(np.float16).view(np.uint8)
    return (x.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)


@pytest.mark.parametrize("gt,rows,width", [(8, 4096, 4096), (1, 4096, 4096), (8, 3, 96), (1, 5, 40), (0, 1, 4096),
                                           (0, 7, 24), (30, 9, 64)])
def test_dequant_bitwise(dev, gt, rows, width):
    from rfill import ops
    rng = np.random.default_rng(gt * 1000 + rows)
    raw = np.ascontiguousarray(_raw(gt, rows, width, rng))
    want = okva.dequant_gguf(raw, gt, width).to(torch.bfloat16)
    got = ops.dequant_gguf_rows(torch.from_numpy(raw).to(dev), gt, width)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))


def test_dequant_strided_and_refusals(dev):
    from rfill import ops
    from rfill._lib import UnsupportedArchitecture
    rng = np.random.default_rng(3)
    raw = gguf_writer.q8_0(6, 64, rng)                           # 68 bytes per row
    pad = np.zeros((6, 80), dtype=np.uint8)
    pad[:, :68] = raw
    out = torch.zeros(6, 72, dtype=torch.bfloat16, device=dev)
    ops.dequant_gguf_rows(torch.from_numpy(pad).to(dev), 8, 64, out=out[:, :64])
    torch.cuda.synchronize()
    assert torch.equal(out[:, :64].cpu(), okva.dequant_gguf(raw, 8, 64).to(torch.bfloat16))
    assert bool((out[:, 64:] == 0).all())
    t = torch.zeros(2, 64, dtype=torch.uint8, device=dev)
    with pytest.raises(UnsupportedArchitecture, match="ggml type 2"):
        ops.dequant_gguf_rows(t, 2, 32)
    with pytest.raises(ValueError, match="multiple of 32"):
        ops.dequant_gguf_rows(t, 8, 48)
    with pytest.raises(ValueError, match="row bytes"):
        ops.dequant_gguf_rows(t, 1, 40)                          # 80 bytes per row needed


def _adapter(path, rng, n=256, bad_dims=False):
    kinds = "full_attention linear_attention full_attention full_attention"
    meta = [("general.architecture", "str", "qwen35"), ("adapter.ridgefill.split", "u32", 1),
            ("adapter.ridgefill.n_embd", "u32", n), ("adapter.ridgefill.model_layer_types", "str", kinds)]
    st = (0.01 * rng.standard_normal((4, 16, 8))).astype(np.float32)     # [heads, V, K]
    w2, w3 = gguf_writer.q8_0(n, n, rng), (np.eye(n) + 0.01 * rng.standard_normal((n, n))).astype(np.float16)
    b2, b3 = (0.001 * rng.standard_normal(n)).astype(np.float32), np.zeros(n, dtype=np.float32)
    ne3 = (n, n // 2) if bad_dims else (n, n)
    tensors = [("blk.1.ridgefill.st", (8, 16, 4), 0, st.tobytes()),
               ("blk.2.ridgefill.weight", (n, n), 8, w2.tobytes()), ("blk.2.ridgefill.bias", (n,), 0, b2.tobytes()),
               ("blk.3.ridgefill.weight", ne3, 1, w3.tobytes()[:ne3[0] * ne3[1] * 2]),
               ("blk.3.ridgefill.bias", (n,), 0, b3.tobytes()),
               ("ridgefill.rowsel.score", (64,), 0, np.zeros(64, np.float32).tobytes())]
    gguf_writer.write(path, meta, tensors)
    return dict(w2=w2, w3=w3, b2=b2, st=st)


def test_load_gguf_adapter(dev, tmp_path):
    from rfill.kva import load_gguf
    rng = np.random.default_rng(4)
    f = _adapter(tmp_path / "ad.gguf", rng)
    proj = load_gguf(tmp_path / "ad.gguf", device=dev)
    torch.cuda.synchronize()
    assert proj.split == 1 and sorted(proj.W) == [2, 3] and proj.meta["native_layers"] == [1]
    assert torch.equal(proj.W[2].cpu(), okva.dequant_gguf(f["w2"], 8, 256).to(torch.bfloat16))
    assert torch.equal(proj.W[3].cpu(), torch.from_numpy(f["w3"].astype(np.float32)).to(torch.bfloat16))
    assert torch.equal(proj.b[2].cpu(), torch.from_numpy(f["b2"]).to(torch.bfloat16))
    assert torch.equal(proj.meta["st"][1], torch.from_numpy(f["st"]).transpose(1, 2))
    x = torch.randn(5, 256, device=dev).to(torch.bfloat16)
    y = proj(2, x)
    ref = x.float() @ proj.W[2].float().T + proj.b[2].float()
    assert float((y.float() - ref).norm() / ref.norm()) < 1e-2


def test_load_gguf_refuses(dev, tmp_path):
    from rfill.kva import load_gguf
    rng = np.random.default_rng(5)
    _adapter(tmp_path / "bad.gguf", rng, bad_dims=True)
    with pytest.raises(ValueError, match="layer 3"):
        load_gguf(tmp_path / "bad.gguf", device=dev)
    gguf_writer.write(tmp_path / "plain.gguf", [("general.architecture", "str", "llama")], [])
    with pytest.raises(ValueError, match="adapter.ridgefill.split"):
        load_gguf(tmp_path / "plain.gguf", device=dev)
