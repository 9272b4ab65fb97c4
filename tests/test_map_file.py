"""The map file format (Projector.save / load / meta_of, check_weights; code/kva/kva.py:121-193), the load-time
hash check (code/kva/integrity.py:179-198), rounded_tail (code/kva/kva.py:270-273) and the per-layer-type fill
selection (Arm.fill_of, code/kva/kva.py:108-115), for the oracle and for the product's host side.

Pins:
  * tests/golden/projector_ref.safetensors was written by the reference's own Projector.save
    (tests/golden/make_projector.py): both loaders read back exactly the bf16 cast of the maps it was given,
    the metadata as strings, and the product's and the oracle's save() write the same header and tensor
    bytes for the same maps;
  * check_weights refuses NaN, +-inf and |w| > 1e4 and accepts 1e4 itself, naming the tensor;
  * a file whose bytes do not match the recorded sha256 is refused, a matching one is loaded and its hash kept;
  * rounded_tail against the reference's own test cases (code/tests/test_tail_round.py:6-17) and a brute
    force over small prompts (the tail is n minus the largest block multiple that leaves >= base rows).
"""
import hashlib
import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import c1  # noqa: E402

from oracle import kva as OK  # noqa: E402
from rfill import integrity  # noqa: E402
from rfill import kva as RK  # noqa: E402


def expected_maps():
    """{layer: [d_out, d_in + 1] bf16}: the fixture maps cast as save() casts them."""
    return {L: torch.cat((w, b[:, None]), 1).to(torch.bfloat16) for L, (w, b) in c1.projector_tensors().items()}


def bits(t):
    return t.contiguous().view(torch.int16)


def test_fixture_pins_the_cast():
    """The fixture holds the round-to-nearest-even cast: 1 + 2^-8 -> 1.0, 1 + 3 2^-8 -> 1 + 2^-6, -0.0 kept."""
    m = expected_maps()[3]
    assert m[0, 0].item() == 1.5 and m[0, 1].item() == 1.0 and m[0, 2].item() == 1.0 + 2.0 ** -6
    assert bits(m[0, 3]).item() == -32768                                    # the sign bit of -0.0
    assert m[1, 0].item() == 9984.0                                          # bf16(1e4)


@pytest.mark.parametrize("loader", ["oracle", "product"])
def test_load_reference_written_file(loader):
    want = expected_maps()
    path = c1.PROJ_FIXTURE
    p = OK.Projector.load(path) if loader == "oracle" else RK.Projector.load(path, "cpu")
    assert p.split == c1.PROJ_SPLIT and sorted(p.W) == sorted(want)
    for L, m in want.items():
        assert p.W[L].dtype == torch.bfloat16 and tuple(p.W[L].shape) == (24, 40)
        assert torch.equal(bits(p.W[L]), bits(m[:, :-1])) and torch.equal(bits(p.b[L]), bits(m[:, -1]))
    assert p.meta == {k: str(v) for k, v in dict(c1.PROJ_META, split=c1.PROJ_SPLIT).items()}
    assert p.sha256 == hashlib.sha256(path.read_bytes()).hexdigest()
    assert RK.Projector.meta_of(path) == p.meta


@pytest.mark.parametrize("writer", ["oracle", "product"])
def test_save_writes_the_reference_bytes(tmp_path, writer):
    """Same maps and metadata -> the file the reference's save() wrote: the same header (tensor names,
    dtypes, shapes, offsets, metadata; safetensors writes the metadata map in hash order, so the header is
    compared parsed) and byte-identical tensor data."""
    maps = c1.projector_tensors()
    W, B = {L: w for L, (w, _) in maps.items()}, {L: b for L, (_, b) in maps.items()}
    cls = OK.Projector if writer == "oracle" else RK.Projector
    out = tmp_path / "p.safetensors"
    cls(c1.PROJ_SPLIT, W, B).save(out, c1.PROJ_META)
    got, ref = out.read_bytes(), c1.PROJ_FIXTURE.read_bytes()
    assert RK._header(got) == RK._header(ref)
    n_got, n_ref = (8 + int.from_bytes(d[:8], "little") for d in (got, ref))
    assert got[n_got:] == ref[n_ref:]


def test_round_trip_between_oracle_and_product(tmp_path):
    g = torch.Generator().manual_seed(41)
    W = {i: torch.randn(32, 16, generator=g).to(torch.bfloat16) for i in (7, 9)}
    B = {i: torch.randn(32, generator=g).to(torch.bfloat16) for i in (7, 9)}
    a, b = tmp_path / "a.safetensors", tmp_path / "b.safetensors"
    RK.Projector(7, W, B).save(a, {"lam": 1e-3})
    OK.Projector(7, W, B).save(b, {"lam": 1e-3})
    for path, cls in ((a, OK.Projector), (b, RK.Projector)):
        p = cls.load(path)
        assert p.split == 7 and p.meta == {"lam": "0.001", "split": "7"}
        for i in W:
            assert torch.equal(bits(p.W[i]), bits(W[i])) and torch.equal(bits(p.b[i]), bits(B[i]))


def test_sha256_checked_on_load(tmp_path):
    path = c1.PROJ_FIXTURE
    sha = hashlib.sha256(path.read_bytes()).hexdigest()
    p = RK.Projector.load(path, "cpu", sha256=sha)
    assert p.sha256 == sha
    wrong = "0" * 64
    with pytest.raises(integrity.IntegrityError):
        RK.Projector.load(path, "cpu", sha256=wrong)
    with pytest.raises(RuntimeError):
        OK.Projector.load(path, sha256=wrong)
    # a file changed after its hash was recorded: refused with the old hash, accepted without one
    changed = tmp_path / "p.safetensors"
    data = bytearray(path.read_bytes())
    data[-1] ^= 0x01                                   # low bit of the last bf16 value's high byte
    changed.write_bytes(bytes(data))
    with pytest.raises(integrity.IntegrityError):
        RK.Projector.load(changed, "cpu", sha256=sha)
    assert RK.Projector.load(changed, "cpu").sha256 == hashlib.sha256(bytes(data)).hexdigest()


@pytest.mark.parametrize("mod", [OK, RK], ids=["oracle", "product"])
@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf"), 1.0001e4, -2e4])
def test_check_weights_refuses(mod, bad):
    t = torch.zeros(5, 7)
    t[3, 2] = bad
    with pytest.raises(ValueError, match="layer.12"):
        mod.check_weights({"layer.11": torch.ones(2, 2), "layer.12": t}, "here")
    ok = torch.zeros(5, 7)
    ok[1, 1], ok[2, 2] = 1e4, -1e4                     # the limit itself is accepted
    mod.check_weights({"layer.12": ok}, "here")


@pytest.mark.parametrize("cls", [OK.Projector, RK.Projector], ids=["oracle", "product"])
def test_save_and_load_refuse_bad_maps(tmp_path, cls):
    from safetensors.torch import save_file
    W = {4: torch.zeros(8, 8)}
    W[4][5, 6] = float("nan")
    with pytest.raises(ValueError, match="layer.4"):
        cls(4, W, {4: torch.zeros(8)}).save(tmp_path / "x.safetensors", {})
    bad = torch.zeros(8, 9, dtype=torch.bfloat16)
    bad[2, 3] = float("inf")
    path = tmp_path / "bad.safetensors"
    save_file({"layer.4": bad}, str(path), metadata={"split": "4"})   # written around save()'s check
    with pytest.raises(ValueError, match="layer.4"):
        cls.load(path)


@pytest.mark.parametrize("fn", [OK.rounded_tail, RK.rounded_tail], ids=["oracle", "product"])
def test_rounded_tail(fn):
    # the reference's own cases (code/tests/test_tail_round.py:6-17)
    assert fn(18984, 4096, 1568) == 18984 - (18984 - 4096) // 1568 * 1568
    assert 4096 <= fn(18984, 4096, 1568) < 4096 + 1568
    assert fn(3000, 4096, 1568) == 3000
    assert fn(4096 + 3 * 1568, 4096, 1568) == 4096
    # brute force: the prefix is the largest block multiple that leaves at least base rows exact
    for base in (1, 5, 16):
        for block in (1, 3, 8):
            for n in range(0, 60):
                start = max([s for s in range(0, n + 1, block) if n - s >= base], default=0)
                assert fn(n, base, block) == n - start, (n, base, block)


def test_fill_of_per_layer_type():
    a = RK.Arm("kva", split=4, tail=8, fill="by_type", fill_by_type=dict(attention="proj", gdn="identity"))
    assert a.fill_of("attn") == "proj" and a.fill_of("gdn") == "identity"
    assert a.uses("identity") and not a.uses("none") and a.prefix_len(20) == 12
    plain = RK.Arm("kva", split=4, tail=8, fill="proj")
    assert plain.fill_of("attn") == plain.fill_of("gdn") == "proj"
    o = OK.Arm("kva", split=4, tail=8, fill="by_type", fill_by_type=dict(attention="oracle", gdn="proj"))
    assert o.fill_of("attn") == "oracle" and o.fill_of("gdn") == "proj"


def test_non_finite_logits_guard():
    x = torch.zeros(3, 4)
    assert RK.check_finite(x, "ok") is x
    for v in (float("nan"), float("inf")):
        y = x.clone()
        y[1, 2] = v
        with pytest.raises(RK.NonFiniteLogits, match="arm x"):
            RK.check_finite(y, "arm x")


def test_refused_arm_options():
    from rfill._lib import UnsupportedArchitecture
    for kw in (dict(f1=True), dict(context=2), dict(rescale="ktail"), dict(fill="kvfold")):
        arm = RK.Arm("a", split=1, tail=4, **{"fill": "proj", **kw})
        with pytest.raises(UnsupportedArchitecture):
            RK._refuse_options(arm)
