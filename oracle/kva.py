"""Oracle fill driver (test infrastructure; see oracle/__init__.py).

Restates the parts of code/kva/kva.py on the fill path: Arm and its prefix length (:79-118), the
Projector map type and its safetensors format (:121-193), rounded_tail (:270-273), run_lower
(:282-300) and finish()'s late-layer loop for the fills 'proj', 'identity', 'oracle' and 'none',
exact rows and the GDN terminal-state correction st (:319-460); and the release's int8 map layout
i8_row128 expanded to bf16 maps (code/c5/convert.py:91-109).
"""
import json
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

MAX_ABS_WEIGHT = 1e4


@dataclass
class Arm:
    name: str
    split: int | None = None
    tail: int = 0
    fill: str = "exact"
    projector: object = None
    st: dict | None = None
    fill_by_type: dict | None = None
    meta: dict = field(default_factory=dict)

    def prefix_len(self, n):
        """P = n - tail (0 for the exact arm), code/kva/kva.py:101-106."""
        return 0 if self.fill == "exact" else max(0, n - self.tail)

    def fill_of(self, layer_type):
        """A late layer's fill: fill_by_type['attention' | 'gdn'] if set, else the arm's (code/kva/kva.py:108-112)."""
        if self.fill_by_type is None:
            return self.fill
        return self.fill_by_type["attention" if layer_type == "attn" else layer_type]


I8_GROUP = 128


def dequant_i8_row128(codes, scale, bias):
    """[rows, width + 1] fp32: codes times their row group's scale, then the bias column
    (code/c5/convert.py:91-97)."""
    rows, width = codes.shape
    if codes.dtype != torch.int8 or width % I8_GROUP or tuple(scale.shape) != (rows, width // I8_GROUP) \
            or tuple(bias.shape) != (rows,):
        raise ValueError(f"i8_row128 shapes {tuple(codes.shape)} {tuple(scale.shape)} {tuple(bias.shape)}")
    w = codes.to(torch.float32).view(rows, width // I8_GROUP, I8_GROUP) * scale.to(torch.float32)[:, :, None]
    return torch.cat([w.view(rows, width), bias.to(torch.float32)[:, None]], 1)


def dequant_gguf(raw, ggml_type, width):
    """fp32 values [rows, width] of a GGUF tensor's raw bytes raw [rows, row_bytes] (numpy uint8), as
    ggml dequantises them: F32 as stored, F16 widened, Q8_0 blocks of 32 (an fp16 scale d, then 32 int8
    codes q) as float(d) * q, BF16 widened (the map tensors of code/qwen38-27b-kit/identity_projector.py:
    26-43, :64-80)."""
    rows = raw.shape[0]
    if ggml_type == 0:
        v = raw.view(np.float32)
    elif ggml_type == 1:
        v = raw.view(np.float16).astype(np.float32)
    elif ggml_type == 30:
        v = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    elif ggml_type == 8:
        blk = raw[:, :width // 32 * 34].reshape(rows, width // 32, 34)
        d = blk[:, :, :2].copy().view(np.float16).astype(np.float32)
        q = blk[:, :, 2:].copy().view(np.int8).astype(np.float32)
        v = (d * q).reshape(rows, width)
    else:
        raise ValueError(f"ggml type {ggml_type}")
    return torch.from_numpy(np.ascontiguousarray(v[:, :width]))


def projector_i8_row128(tensors, split):
    """The Projector of the i8_row128 tensors proj.L.{codes, scale, bias}: each layer's [d_out, d_in + 1]
    map cast to bf16 once (code/c5/convert.py:100-109), weight and bias columns split as Projector.load."""
    W, B = {}, {}
    for L in sorted({int(k.split(".")[1]) for k in tensors if k.endswith(".codes")}):
        m = dequant_i8_row128(tensors[f"proj.{L}.codes"], tensors[f"proj.{L}.scale"],
                              tensors[f"proj.{L}.bias"]).to(torch.bfloat16)
        W[L], B[L] = m[:, :-1].contiguous(), m[:, -1].contiguous()
    return Projector(split, W, B, {"layout": "i8_row128"})


def rounded_tail(n, base, block):
    """Tail length when the prefix boundary is rounded down to a block multiple (code/kva/kva.py:270-273)."""
    start = max(0, (n - base) // block * block)
    return n - start


def check_weights(tensors, where):
    """Refuse stored maps with a non-finite entry or |w| > 1e4 (code/kva/kva.py:121-134)."""
    for name, t in tensors.items():
        tf = t.float()
        bad = ~torch.isfinite(tf) | (tf.abs() > MAX_ABS_WEIGHT)
        if bool(bad.any()):
            r, c = bad.nonzero()[0].tolist()
            raise ValueError(f"{where}: {name} has {int(bad.sum())} non-finite or |w| > {MAX_ABS_WEIGHT:g} "
                             f"weights (first at row {r}, col {c}); refusing")


class Projector:
    """x_i = b W_i^T + c_i per late layer (code/kva/kva.py:137-156). File format (:161-193):
    safetensors, tensor 'layer.{i}' = [d_out, d_in + 1] bf16 with the bias as the last column, string
    metadata including 'split'."""

    def __init__(self, split, weights, biases, meta=None):
        self.split, self.W, self.b, self.meta = split, weights, biases, meta or {}

    def __call__(self, i, b):
        return F.linear(b, self.W[i].to(b.dtype), self.b[i].to(b.dtype))

    def save(self, path, meta):
        from safetensors.torch import save_file
        out = {f"layer.{i}": torch.cat((self.W[i], self.b[i][:, None]), 1).to(torch.bfloat16).contiguous()
               for i in sorted(self.W)}
        check_weights(out, f"Projector.save {path}")
        save_file(out, str(path), metadata={k: str(v) for k, v in dict(meta, split=self.split).items()})

    @classmethod
    def load(cls, path, dtype=torch.bfloat16, sha256=None):
        """Maps from the file's bytes, read once; with sha256 given, bytes of another hash are refused
        (code/kva/kva.py:161-178; the page-cache re-read of code/kva/integrity.py is the product's)."""
        import hashlib
        from safetensors.torch import load as from_bytes
        with open(path, "rb") as f:
            data = f.read()
        sha = hashlib.sha256(data).hexdigest()
        if sha256 is not None and sha != sha256:
            raise RuntimeError(f"{path}: sha256 {sha}, expected {sha256}")
        meta = json.loads(data[8:8 + int.from_bytes(data[:8], "little")]).get("__metadata__") or {}
        W, B = {}, {}
        for name, t in from_bytes(data).items():
            check_weights({name: t}, f"Projector.load {path}")
            i = int(name.split(".")[1])
            W[i], B[i] = t[:, :-1].to(dtype).contiguous(), t[:, -1].to(dtype).contiguous()
        p = cls(int(meta["split"]), W, B, meta)
        p.sha256 = sha
        return p


def run_lower(model, ids, splits):
    """Exact forward of layers < max(splits); returns ({split: h_split}, cache) (code/kva/kva.py:282-300)."""
    pos = torch.arange(ids.shape[0])
    cache = model.new_cache()
    h = model.embed(ids)
    hs = {}
    for i in range(max(splits)):
        if i in splits:
            hs[i] = h
        h = model.layer(i, h, pos, cache)
    hs[max(splits)] = h
    return hs, cache


def finish(model, ids, h_split, lower_cache, arm, keep, oracle=None, exact_rows=None, fill_store=None,
           row_inputs=None, fill_reuse=None, keep_cache=True, hook=None):
    """Late layers of one arm (code/kva/kva.py:319-460, the fill subset). Prefix rows [0, P) fill each
    late layer from x (projector / identity / true inputs, per layer type through fill_by_type) with the
    exact rows R scattered in (index_copy) and run through layer_rows -- or, with fill 'none', only the
    rows R run the layer; a fill_reuse dict replaces the fill; then +st; then the tail rows run the exact
    layer (hook(i, h) first; keep_cache=False drops the layer's cache after).
    row_inputs (dict): receives the exact rows' input to every late layer {layer: [|R|, H]}.
    Returns (logits of the last `keep` rows, cache, P)."""
    n = ids.shape[0]
    split = arm.split
    P = arm.prefix_len(n)
    pos = torch.arange(n)
    cache = [dict(c) for c in lower_cache[:split]] + [dict() for _ in range(model.n_layers - split)]
    if keep > n - P:
        raise ValueError(f"keep {keep} rows > exact tail {n - P}")
    b, h = h_split[:P], h_split[P:]
    rows = None
    if exact_rows is not None and len(exact_rows) > 0:
        rows = torch.as_tensor(exact_rows, dtype=torch.long)
        if int(rows[-1]) >= P or bool((rows.diff() <= 0).any()):
            raise ValueError("exact rows: sorted unique rows < P")
        hr = h_split[rows]
    if rows is not None and fill_reuse is not None:
        raise ValueError("exact rows: no fill reuse")
    for i in range(split, model.n_layers):
        fill = arm.fill_of(model.layer_types[i])
        if P > 0 and fill_reuse is not None:
            if fill_reuse[i].get("n", P) != P:
                raise ValueError(f"reused fill of layer {i} has {fill_reuse[i]['n']} rows, P = {P}")
            cache[i] = dict(fill_reuse[i])
        elif P > 0:
            if fill == "none":
                if rows is not None:
                    if row_inputs is not None:
                        row_inputs[i] = hr
                    hr = model.layer(i, hr, pos[rows], cache)
            else:
                if fill == "proj":
                    x = arm.projector(i, b)
                elif fill == "identity":
                    x = b
                elif fill == "oracle":
                    x = oracle[i][:P]
                else:
                    raise ValueError(fill)
                if rows is not None:
                    if row_inputs is not None:
                        row_inputs[i] = hr
                    x = x.index_copy(0, rows, hr.to(x.dtype))
                    hr = model.layer_rows(i, x, pos[:P], rows, cache)
                else:
                    model.fill(i, x, pos[:P], cache)
        if P > 0 and fill_store is not None:
            fill_store[i] = dict(cache[i])
        st = arm.st.get(i) if (arm.st and P > 0) else None
        if st is not None:
            cache[i]["rec"] = cache[i]["rec"] + st.to(cache[i]["rec"])
        if hook is not None:
            hook(i, h)
        h = model.layer(i, h, pos[P:], cache)
        if not keep_cache:
            cache[i] = {}
    return model.logits(h[h.shape[0] - keep:]), cache, P
