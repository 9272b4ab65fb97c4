"""Fill driver over the device fill model: the reference's Arm, Projector map type, run_lower and finish()
(code/kva/kva.py:79-193, 282-300, 319-460), with every fill step on librfill kernels.

fill_late() runs the hot path of finish() for one arm: for each late layer i >= split, the prefix rows
[0, P) get the layer's fill (Arm.fill_of: the arm's fill, or per layer type through fill_by_type) --
x_i = W_i b + c_i ('proj', one rf_map_apply that also yields x's RMSNorm statistics), x_i = b
('identity'), the true inputs ('oracle') or nothing ('none') -- the exact rows R are scattered in
bit-exactly (rf_row_scatter, the index_copy of kva.py:428-431), the layer's cache is filled
(rf_norm_kv_write, or the GDN fill) and, for exact rows, the layer's full computation runs on them
(FillModel.layer_rows, kva.py:436-437) to give their next input. Two x / statistics buffers and one RoPE
table serve all late layers; optionally layer i's cache work runs on a second stream beside layer i + 1's
map apply (two_stream). finish() adds fill reuse, the st corrections, the exact tail and the logits.
"""
import json
from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops

MAX_ABS_WEIGHT = 1e4

# Fills this package runs per late layer; the other fills of the reference are refused by name.
FILLS = ("proj", "identity", "oracle", "none")
UNSUPPORTED_FILLS = ("swiftkv", "swiftkv_native", "kvfold")


class NonFiniteLogits(RuntimeError):
    """Logits with a NaN or an infinity: a broken forward stops the run rather than becoming a data point
    (code/kva/kva.py:470-473)."""


def check_finite(logits, where):
    """logits unchanged if every entry is finite, else NonFiniteLogits naming `where` (code/kva/kva.py:476-479)."""
    if not bool(torch.isfinite(logits).all()):
        raise NonFiniteLogits(f"{where}: logits hold NaN or infinite values")
    return logits


@dataclass
class Arm:
    """An arm's fill parameters (code/kva/kva.py:79-118). The fields are the reference's, so arms built for
    it build here too. finish() runs the fills in FILLS, per layer type through fill_by_type
    ({'attention': fill, 'gdn': fill}), with exact rows, st corrections and fill reuse; the exploratory
    options (f1, kvfold, context, refresh, tail_bias_from, exact_part, rescale) are refused by name."""
    name: str
    split: int | None = None
    tail: int = 0
    fill: str = "exact"
    projector: object = None
    st: dict | None = None
    f1: bool = False
    fill_by_type: dict | None = None
    kvfold: object = None
    context: int = 0
    refresh: int | None = None
    refresh_projector: object = None
    tail_bias_from: int | None = None
    tail_bias_skip_last: int = 0
    exact_part: str | None = None
    rescale: str | None = None
    rescale_skip_last: int = 0
    tail_from: str | None = None
    meta: dict = field(default_factory=dict)

    def prefix_len(self, n):
        if self.fill == "exact":
            return 0
        if self.fill == "swiftkv_native":
            return n
        return max(0, n - self.tail)

    def fill_of(self, layer_type):
        """The fill of a late layer of type 'attn' or 'gdn' (fill_by_type names them 'attention' and 'gdn')."""
        if self.fill_by_type is None:
            return self.fill
        return self.fill_by_type["attention" if layer_type == "attn" else layer_type]

    def uses(self, fill):
        return fill in (self.fill_by_type.values() if self.fill_by_type else (self.fill,))


def _refuse_options(arm):
    """UnsupportedArchitecture for an arm option outside the fill path built here."""
    from ._lib import UnsupportedArchitecture
    opts = dict(f1=arm.f1, kvfold=arm.kvfold is not None, context=arm.context, refresh=arm.refresh is not None,
                tail_bias_from=arm.tail_bias_from is not None, exact_part=arm.exact_part is not None,
                rescale=arm.rescale is not None)
    on = [k for k, v in opts.items() if v]
    if on:
        raise UnsupportedArchitecture(f"arm {arm.name!r}: option(s) {', '.join(on)} are not implemented on the device")
    for f in (arm.fill_by_type or {}).values() if arm.fill_by_type else (arm.fill,):
        if f in UNSUPPORTED_FILLS:
            raise UnsupportedArchitecture(f"arm {arm.name!r}: fill {f!r} is not implemented on the device")


def rounded_tail(n, base, block):
    """Exact-tail length of an n-row prompt when a block-granular scheduler rounds the prefix boundary down
    to a multiple of `block` with at least `base` rows left exact: the boundary is the largest block multiple
    <= n - base (0 if n < base), so base <= tail < base + block for long prompts (code/kva/kva.py:270-273)."""
    return n - max(0, (n - base) // block * block)


def check_weights(tensors, where):
    """Refuse stored maps {name: [d_out, d_in + 1]} that hold a NaN, an infinity or an entry of magnitude
    above MAX_ABS_WEIGHT -- what a failed fit, or bytes damaged after the file was written, leave behind.
    Raises ValueError naming the tensor and its first bad entry (the refusal of code/kva/kva.py:121-134)."""
    for name, t in tensors.items():
        v = t.float()
        ok = torch.isfinite(v) & (v.abs() <= MAX_ABS_WEIGHT)
        if bool(ok.all()):
            continue
        bad = (~ok).nonzero()
        at = tuple(bad[0].tolist())
        raise ValueError(f"{where}: refusing {name}: {bad.shape[0]} entries are NaN, infinite or above "
                         f"{MAX_ABS_WEIGHT:g} in magnitude, the first at {list(at)} = {v[at].item():.4g}")


def _header(data):
    """The JSON header of safetensors bytes."""
    n = int.from_bytes(data[:8], "little")
    return json.loads(data[8:8 + n])


class Projector:
    """Per late layer x_i = b W_i^T + c_i in bf16 (code/kva/kva.py:137-159). Maps may live anywhere;
    the first call on a GPU keeps one bf16 device copy (release() drops it). File format
    (code/kva/kva.py:161-193): safetensors, 'layer.{i}' = [d_out, d_in + 1] bf16, bias last column,
    string metadata with 'split'; load() checks the file's sha256 and keeps it as .sha256."""

    def __init__(self, split, weights, biases, meta=None):
        self.split, self.W, self.b, self.meta = split, weights, biases, meta or {}
        self._dev = None
        self.sha256 = None

    def _maps(self, device):
        if self._dev is None or self._dev[0] != device:
            self._dev = (device,
                         {i: w.to(device, torch.bfloat16).contiguous() for i, w in self.W.items()},
                         {i: c.to(device, torch.bfloat16).contiguous() for i, c in self.b.items()})
        return self._dev[1], self._dev[2]

    def apply(self, i, b, out=None, ssq=None, workspace=None):
        """(x_i [P, d_out] bf16, its row sum-of-squares partials) for rows b [P, d_in] bf16. workspace: the
        GEMM's split-K workspace (ops.map_apply)."""
        W, B = self._maps(b.device)
        return ops.map_apply(b, W[i], B[i], out, ssq, workspace=workspace)

    def apply_batch(self, ids, b, outs, ssqs):
        """apply() of several layers in one launch (ops.map_apply_batch): outs[k] / ssqs[k] receive layer ids[k]'s
        x and row statistics, bit-identical to apply() of it alone without a workspace."""
        W, B = self._maps(b.device)
        ops.map_apply_batch(b, [W[i] for i in ids], [B[i] for i in ids], outs, ssqs)

    def __call__(self, i, b):
        return self.apply(i, b)[0]

    def release(self):
        self._dev = None

    def save(self, path, meta):
        """Write the maps as [W | c] cast once to bf16 (the two operands promoted to one dtype first, so a
        map saved here is the same file the reference writes for the same tensors), refusing bad maps."""
        from safetensors.torch import save_file
        out = {}
        for i in sorted(self.W):
            w, c = self.W[i], self.b[i].to(self.W[i].device)
            out[f"layer.{i}"] = torch.cat((w, c[:, None]), 1).to(torch.bfloat16).cpu().contiguous()
        check_weights(out, f"Projector.save {path}")
        save_file(out, str(path), metadata={k: str(v) for k, v in dict(meta, split=self.split).items()})

    @staticmethod
    def meta_of(path):
        """The file's string metadata from its header alone (no maps read)."""
        with open(path, "rb") as f:
            n = int.from_bytes(f.read(8), "little")
            return json.loads(f.read(n)).get("__metadata__") or {}

    @classmethod
    def load(cls, path, device="cpu", dtype=torch.bfloat16, sha256=None):
        """The maps of a file written by save(): the bytes are read once and checked against sha256 (the
        hash recorded when the file was written; None: the disk copy, read around the page cache), and
        the maps come from those same bytes. Refuses bad maps (check_weights)."""
        from safetensors.torch import load as from_bytes
        from .integrity import read_verified
        data, sha = read_verified(path, sha256)
        meta = _header(data).get("__metadata__") or {}
        W, B = {}, {}
        for name, t in from_bytes(data).items():
            check_weights({name: t}, f"Projector.load {path}")
            i = int(name.split(".")[1])
            W[i] = t[:, :-1].to(device, dtype).contiguous()
            B[i] = t[:, -1].to(device, dtype).contiguous()
        p = cls(int(meta["split"]), W, B, meta)
        p.sha256 = sha
        return p


I8_GROUP = 128


def load_i8_row128(tensors, split, device="cuda"):
    """Projector from the i8_row128 maps of the public release (code/c5/convert.py:4-23): for each late
    layer L, proj.L.codes int8 [d_out, d_in], proj.L.scale bf16 [d_out, d_in / 128] (row i's 128-column
    group g is codes[i, 128 g : 128 g + 128] * scale[i, g]) and proj.L.bias bf16 [d_out]. tensors: a dict
    of those tensors (e.g. safetensors.torch.load_file of the release's proj8 files) or a list of file
    paths. The maps are expanded on the device by rf_dequant_i8_rows: codes * scale in fp32 (exact), one
    cast to bf16, as convert.py's dequant + .to(bfloat16) (:91-109); the bias stays the release's bf16."""
    if not isinstance(tensors, dict):
        from safetensors.torch import load_file
        merged = {}
        for path in tensors:
            merged.update(load_file(str(path)))
        tensors = merged
    layers = sorted({int(k.split(".")[1]) for k in tensors if k.startswith("proj.") and k.endswith(".codes")})
    if not layers:
        raise ValueError("load_i8_row128: no proj.<L>.codes tensors")
    device = torch.device(device)
    W, B = {}, {}
    for L in layers:
        try:
            codes, scale, bias = (tensors[f"proj.{L}.{k}"] for k in ("codes", "scale", "bias"))
        except KeyError as e:
            raise ValueError(f"load_i8_row128: layer {L} lacks {e.args[0]}") from None
        rows, width = codes.shape
        if (codes.dtype != torch.int8 or scale.dtype != torch.bfloat16 or bias.dtype != torch.bfloat16
                or width % I8_GROUP or tuple(scale.shape) != (rows, width // I8_GROUP) or tuple(bias.shape) != (rows,)):
            raise ValueError(f"load_i8_row128: layer {L} shapes codes {tuple(codes.shape)} {codes.dtype}, scale "
                             f"{tuple(scale.shape)} {scale.dtype}, bias {tuple(bias.shape)} {bias.dtype}")
        W[L] = ops.dequant_i8_rows(codes.to(device).contiguous(), scale.to(device).contiguous(), I8_GROUP)
        B[L] = bias.to(device).contiguous()
        check_weights({f"layer.{L}": W[L]}, "load_i8_row128")
    return Projector(split, W, B, {"layout": "i8_row128"})


def load_gguf(path, device="cuda"):
    """The Projector of a llama.cpp adapter file (the GGUF maps of code/qwen38-27b-kit/identity_projector.py:
    15-80): metadata adapter.ridgefill.split, .n_embd and .model_layer_types; for each late attention
    layer L, blk.L.ridgefill.weight (F16, Q8_0, F32 or BF16, ne = [n_in, n_out]) expanded to bf16 on the
    device (rf_dequant_gguf_rows) and blk.L.ridgefill.bias (F32) cast to bf16. Linear-attention layers
    carry no map (the engine feeds them h_S itself); they are listed in meta["native_layers"] and their
    blk.L.ridgefill.st corrections, read in the engines' [heads, V, K] order, are returned by
    st_from_engine in meta["st"]. The metadata entries are kept in meta as strings."""
    from . import gguf
    fields, tensors = gguf.read(path)
    for k in ("adapter.ridgefill.split", "adapter.ridgefill.n_embd", "adapter.ridgefill.model_layer_types"):
        if k not in fields:
            raise ValueError(f"{path}: metadata {k!r} missing (not a RidgeFill adapter)")
    split, n = int(fields["adapter.ridgefill.split"]), int(fields["adapter.ridgefill.n_embd"])
    kinds = str(fields["adapter.ridgefill.model_layer_types"]).split()
    W, B, native, st = {}, {}, [], {}
    dev = torch.device(device)

    def expand(t, rows, width):
        raw = torch.from_numpy(np.array(t.data)).to(dev)
        return ops.dequant_gguf_rows(raw, t.ggml_type, width).view(rows, width)

    for L in range(split, len(kinds)):
        base = f"blk.{L}.ridgefill."
        if kinds[L] == "linear_attention":
            native.append(L)
            if base + "st" in tensors:
                t = tensors[base + "st"]
                if t.ggml_type != gguf.GGML_F32 or len(t.ne) != 3:
                    raise ValueError(f"{path}: {base}st must be F32 [heads, V, K]")
                st[L] = torch.from_numpy(np.array(t.data).view(np.float32).reshape(t.shape))
            continue
        w, b = tensors.get(base + "weight"), tensors.get(base + "bias")
        if w is None or b is None:
            raise ValueError(f"{path}: layer {L} ({kinds[L]}) has no {base}weight / {base}bias")
        if len(w.ne) != 2 or w.ne[0] != n or b.ne != (w.ne[1],) or b.ggml_type != gguf.GGML_F32:
            raise ValueError(f"{path}: layer {L}: weight dims {w.ne} (expected [{n}, n_out]), bias dims {b.ne} "
                             f"type {b.ggml_type} (expected F32 [n_out])")
        W[L] = expand(w, w.ne[1], w.ne[0])
        B[L] = expand(b, 1, b.ne[0]).view(-1)
    check_weights({f"layer.{L}": torch.cat((W[L].float(), B[L].float()[:, None]), 1) for L in W}, str(path))
    meta = {k: str(v) for k, v in fields.items() if k.startswith("adapter.") or k == "general.architecture"}
    meta.update(split=str(split), native_layers=native, st=st_from_engine(st) if st else {})
    return Projector(split, W, B, meta)


def adapter_arm(name, projector, tail):
    """The arm a llama.cpp adapter drives (code/qwen38-27b-kit/identity_projector.py:15-80): a Projector from
    load_gguf fills the layers it has maps for; the layers the engine runs natively (the linear-attention,
    i.e. GDN, layers) take h_S itself, the 'identity' fill, and their st corrections. A projector with no
    native layers gives the plain 'proj' arm."""
    native = projector.meta.get("native_layers") or []
    st = projector.meta.get("st") or None
    if not native:
        return Arm(name, split=projector.split, tail=tail, fill="proj", projector=projector, st=st)
    return Arm(name, split=projector.split, tail=tail, fill="by_type", projector=projector, st=st,
               fill_by_type={"attention": "proj", "gdn": "identity"})


def st_from_engine(st):
    """GDN terminal-state corrections in the engines' layout [heads, V, K] (code/c5/convert.py:7-8) to
    the fill's recurrent-state layout [heads, dk, dv] (code/kva/ops.py:4-6, Qwen35.fill's rec += st):
    {L: [h, V, K]} -> {L: [h, K, V]} fp32."""
    out = {}
    for L, t in st.items():
        if t.dim() != 3:
            raise ValueError(f"st_from_engine: layer {L} shape {tuple(t.shape)} (expected [heads, V, K])")
        out[int(L)] = t.transpose(1, 2).to(torch.float32).contiguous()
    return out


def check_rows(exact_rows, P):
    """Sorted unique int64 rows < P, else ValueError (code/kva/kva.py:357-362)."""
    rows = torch.as_tensor(exact_rows, dtype=torch.long)
    if rows.dim() != 1 or rows.numel() == 0:
        raise ValueError("exact rows: a non-empty 1-d row list")
    rc = rows.cpu()
    if int(rc[-1]) >= P or int(rc[0]) < 0 or bool((rc.diff() <= 0).any()):
        raise ValueError("exact rows: sorted unique rows < P")
    return rows


def two_stream(layers, produce, consume, device):
    """Run produce(i, slot) for each layer on the current stream and consume(i, slot) on a second
    stream (default priority), slot = position % 2 naming one of two buffer sets: consume(i) waits for
    produce(i), and produce(i + 2) waits for consume(i) before reusing its slot. The second stream's
    K / V GEMM of layer i thus overlaps the map GEMM of layer i + 1 (their tile counts do not fill the
    GPU's last wave alike). Returns after the current stream has been ordered after all of it."""
    main = torch.cuda.current_stream(device)
    side = torch.cuda.Stream(device=device)
    side.wait_stream(main)
    ready = [torch.cuda.Event(), torch.cuda.Event()]
    free = [torch.cuda.Event(), torch.cuda.Event()]
    for n, i in enumerate(layers):
        slot = n % 2
        if n >= 2:
            main.wait_event(free[slot])
        produce(i, slot)
        ready[slot].record(main)
        side.wait_event(ready[slot])
        with torch.cuda.stream(side):
            consume(i, slot)
        free[slot].record(side)
    main.wait_stream(side)


# Consecutive attention layers filled together by fill_late (one map launch, then one K / V launch per group).
ATTN_GROUP = 4
# a hybrid stack's groups (GDN and attention layers): 8 layers, so that the group's GDN fills pair up (the
# Qwen3.5 pattern of 3 GDN + 1 attention leaves one unpaired GDN layer in every 4)
HYBRID_GROUP = 8


def serial(layers, produce, consume, device, pair=None, group=None):
    """produce(i, slot) then consume(i, slot) for each layer, all on the current stream. pair: (can(i, j),
    consume_pair(i, slot_i, j, slot_j)): two consecutive layers with can(i, j) are produced both, then
    consumed together. group: (size, can(i), run(ids)): a run of 2 .. size consecutive layers with can(i)
    goes to run(ids), which produces and consumes them itself."""
    n, k = 0, 0
    while k < len(layers):
        i = layers[k]
        if group is not None and group[1](i):
            m = 1
            while m < group[0] and k + m < len(layers) and group[1](layers[k + m]):
                m += 1
            if m > 1:
                group[2](layers[k:k + m])
                k += m
                continue
        if pair is not None and k + 1 < len(layers) and pair[0](i, layers[k + 1]):
            j = layers[k + 1]
            produce(i, n % 2)
            produce(j, (n + 1) % 2)
            pair[1](i, n % 2, j, (n + 1) % 2)
            n, k = n + 2, k + 2
            continue
        produce(i, n % 2)
        consume(i, n % 2)
        n, k = n + 1, k + 1


def _layer_fill(arm, model, i):
    """The fill of late layer i for this arm, checked against the fills this package runs."""
    f = arm.fill_of(model.layer_types[i])
    if f not in FILLS:
        from ._lib import UnsupportedArchitecture
        if f in UNSUPPORTED_FILLS:
            raise UnsupportedArchitecture(f"fill {f!r} (layer {i}) is not implemented on the device")
        raise ValueError(f"fill {f!r} (layer {i}): expected one of {FILLS}")
    return f


def fill_late(model, h_split, arm, exact_rows=None, hr=None, cache=None, overlap=False, row_inputs=None, oracle=None):
    """The late-layer fill of finish() for one arm: every late layer's cache filled from the prefix rows
    [0, P) of h_split [N, H] (bf16, on the GPU), with exact rows R (sorted prefix rows) whose inputs replace
    the fill's x (code/kva/kva.py:392-454). Each late layer takes its arm's fill for its type (Arm.fill_of):
    'proj' x = W_i b + c_i, 'identity' x = b, 'oracle' x = oracle[i][:P] (given true inputs), 'none' no
    prefix fill (with exact rows, the rows alone run the layer: code/kva/kva.py:406-411).

    hr None (the reference's path): the rows enter the first late layer with their split-layer state
    h_split[R]; each late layer fills its cache with them scattered in and runs its full layer on them
    (layer_rows), whose output is their input to the next layer. hr given (one [|R|, H] tensor for every
    layer, or {layer: tensor}): those inputs are scattered in and no full layer runs.
    row_inputs (dict): receives the rows' input to every late layer. overlap: run each layer's cache work
    on a second stream beside the next layer's map apply (two_stream). Returns (cache, P)."""
    n = h_split.shape[0]
    P = arm.prefix_len(n)
    cache = model.new_cache() if cache is None else cache
    if arm.fill == "exact":
        raise ValueError("fill 'exact' has no prefix fill")
    _refuse_options(arm)
    layers = list(range(arm.split, model.n_layers))
    fills = {i: _layer_fill(arm, model, i) for i in layers}
    if P == 0:
        return cache, P
    dev = h_split.device
    b = h_split[:P]
    pos = torch.arange(P, device=dev)
    cs = model.rope_table(pos)
    rows = None
    if exact_rows is not None and len(exact_rows) > 0:
        rows = check_rows(exact_rows, P).to(dev)
    computed = rows is not None and hr is None
    if hr is not None and "none" in fills.values():
        raise ValueError("fill 'none' runs the exact rows' layers itself; it takes no given row inputs")
    if oracle is None and "oracle" in fills.values():
        raise ValueError("fill 'oracle' fills from the true late-layer inputs: pass oracle={layer: [>= P, H]}")
    H = h_split.shape[1]
    for i in layers:                                    # allocate / grow every cache before any launch
        if model.layer_types[i] == "attn":
            model.reserve(cache[i], rows.shape[0] if fills[i] == "none" and rows is not None else P,
                          model.n_kv, model.head_dim, dev)
    xbuf = [torch.empty(P, H, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    sbuf = [torch.empty(P, ops.ssq_parts(H), dtype=torch.float32, device=dev) for _ in range(2)]
    base_ssq = (ops.row_ssq(b) if rows is None and "identity" in fills.values() else None)
    # attention-only stacks filled by their maps: the fill of a layer reads the exact rows only at their own
    # slots, so every layer is filled first (grouped, as without rows) and the rows then overwrite their
    # K / V layer by layer (FillModel.rows_over_fill); GDN layers carry the rows' inputs into later states
    decoupled = (computed and not overlap and all(model.layer_types[i] == "attn" and fills[i] == "proj"
                                                  for i in layers))
    g0 = ops.row_gather(b, rows) if computed else (None, None)
    state = {"hr": g0[0], "sr": g0[1]}
    qpos = rows if rows is not None else None
    inputs = {}

    def produce(i, slot):
        f = fills[i]
        if f == "none":
            inputs[slot] = None
            return
        if f == "proj":
            W = arm.projector._maps(dev)[0][i]
            x, ssq = arm.projector.apply(i, b, xbuf[slot], sbuf[slot],
                                         workspace=model.gemm_workspace(P, W.shape[0], W.shape[1], dev, "produce"))
        elif f == "identity" and rows is None:
            x, ssq = b, base_ssq
        else:
            src = b if f == "identity" else oracle[i][:P]
            if src.shape != b.shape:
                raise ValueError(f"oracle inputs of layer {i}: shape {tuple(src.shape)}, expected {tuple(b.shape)}")
            x = xbuf[slot].copy_(src)
            ssq = ops.row_ssq(x, sbuf[slot])
        if rows is not None and not computed:
            hri = (hr[i] if isinstance(hr, dict) else hr).to(dev, torch.bfloat16)
            if row_inputs is not None:
                row_inputs[i] = hri
            ops.row_scatter(x, ssq, rows, hri)
        inputs[slot] = (x, ssq)

    def consume(i, slot):
        if fills[i] == "none":
            if rows is not None:                        # only the exact rows reach this layer
                if row_inputs is not None:
                    row_inputs[i] = state["hr"]
                state["hr"] = model.layer(i, state["hr"], qpos, cache)[0]
            return
        x, ssq = inputs[slot]
        if computed and not decoupled:
            if row_inputs is not None:
                row_inputs[i] = state["hr"]
            ops.row_scatter(x, ssq, rows, state["hr"])
            if i == layers[-1]:                         # the rows' output past the last late layer is unused
                model.fill(i, x, pos, cache, ssq=ssq, cs=cs)
            else:
                state["hr"] = model.layer_rows(i, x, pos, rows, cache, ssq=ssq, cs=cs)
        else:
            model.fill(i, x, pos, cache, ssq=ssq, cs=cs)

    def can_pair(i, j):                                 # two GDN layers whose fills do not wait on exact rows
        return (not computed and model.layer_types[i] == "gdn" and model.layer_types[j] == "gdn"
                and fills[i] != "none" and fills[j] != "none")

    def consume_pair(i, si, j, sj):
        (xi, qi), (xj, qj) = inputs[si], inputs[sj]
        model.fill_batch([i, j], [xi, xj], cache, ssqs=[qi, qj])

    gbuf = []

    def can_group(i):                                   # layers filled by their maps, no rows computed between
        return (not computed or decoupled) and fills[i] == "proj"

    def run_group(ids):
        """The maps of several late layers in one launch (the GEMM fills whole waves of the GPU, with no tail
        per layer), then the group's attention layers' K / V fills in one launch and its GDN layers' fills in
        pairs (any two: the layers' fills are independent), each pair's in-projections in one launch right
        before its delta-rule fill; each layer's results are bit-identical to its unsplit map apply and fill
        alone."""
        while len(gbuf) < len(ids):
            gbuf.append((torch.empty(P, H, dtype=torch.bfloat16, device=dev),
                         torch.empty(P, ops.ssq_parts(H), dtype=torch.float32, device=dev)))
        xs, ss = [g[0] for g in gbuf[:len(ids)]], [g[1] for g in gbuf[:len(ids)]]
        arm.projector.apply_batch(ids, b, xs, ss)
        if rows is not None and not computed:           # given row inputs
            for i, x, q in zip(ids, xs, ss):
                hri = (hr[i] if isinstance(hr, dict) else hr).to(dev, torch.bfloat16)
                if row_inputs is not None:
                    row_inputs[i] = hri
                ops.row_scatter(x, q, rows, hri)
        attn = [k for k, i in enumerate(ids) if model.layer_types[i] == "attn"]
        if attn:
            model.fill_attn_batch([ids[k] for k in attn], [xs[k] for k in attn], pos, cache,
                                  ssqs=[ss[k] for k in attn], cs=cs)
        gdn = [k for k, i in enumerate(ids) if model.layer_types[i] == "gdn"]
        for j in range(0, len(gdn), 2):                 # each pair's in-projections, then its fill: the
            ks = gdn[j:j + 2]                           # projected rows are read back while still cached
            model.fill_batch([ids[k] for k in ks], [xs[k] for k in ks], cache, ssqs=[ss[k] for k in ks])

    if overlap:
        two_stream(layers, produce, consume, dev)
    else:
        gsize = HYBRID_GROUP if any(model.layer_types[i] == "gdn" for i in layers) else ATTN_GROUP
        serial(layers, produce, consume, dev, pair=(can_pair, consume_pair), group=(gsize, can_group, run_group))
    if decoupled:
        # every layer is filled from the prefix rows' map outputs; the rows now run their layers in order, each
        # overwriting its own K / V slots (their inputs replace the fill's at those rows only)
        hr_i, sr_i = state["hr"], state["sr"]
        qp = pos[rows]
        for i in layers:
            if row_inputs is not None:
                row_inputs[i] = hr_i
            out = model.rows_over_fill(i, hr_i, sr_i, pos, rows, cache, cs, full=i != layers[-1], rows_max=P - 1,
                                       qpos=qp)
            if out is not None:
                hr_i, sr_i = out
        state["hr"] = hr_i
    return cache, P


def run_lower(model, ids, splits):
    """Exact forward of the layers below max(splits) over all prompt rows (code/kva/kva.py:282-300):
    ({split: h_split [N, H] bf16}, cache with those layers filled). model needs its lower layers packed."""
    splits = set(splits)
    top = max(splits)
    got = {}

    def hook(i, h):
        if i in splits:
            got[i] = h

    cache = model.new_cache()
    if top == 0:
        got[0] = model.embed(ids)[0]
        return got, cache
    _, cache = model.forward_exact(ids, hook=hook, cache=cache, stop=top)
    return got, cache


def finish(model, ids, h_split, lower_cache, arm, keep, oracle=None, keep_cache=True, fill_store=None,
           fill_reuse=None, exact_rows=None, row_inputs=None, hook=None, mix=None, hr=None):
    """Layers >= arm.split for one arm, as finish() runs them (code/kva/kva.py:319-460), with the reference's
    call signature: ids [N] (only its length is read here), h_split [N, H] (moved to the model's device as
    bf16), lower_cache (the caches of layers < split from run_lower, kept; None for a model packed with its
    late layers only), keep (the last rows whose logits to return), oracle ({layer: true inputs [>= P, H]}
    for 'oracle' fills), keep_cache=False (each late layer's cache is dropped once the tail has run it),
    fill_store (dict: receives each late layer's cache right after its prefix fill, before + st), fill_reuse
    (such a dict from an arm with the same fill, split and P: used instead of filling), exact_rows and
    row_inputs (as fill_late), hook(i, h) (the tail's rows before layer i runs). mix feeds context arms,
    which are refused. hr: given exact-row inputs (fill_late's hr), an addition to the reference's API.

    Every late layer's cache is filled from the prefix rows [0, P) first (fill_late), then the exact tail
    [P, N) runs through each late layer in order (FillModel.layer over that layer's filled cache,
    kva.py:457). The fill of a layer never reads the tail, so this gives the reference's interleaved order's
    results. Attention caches are sized once for all N rows. arm.st {layer: [heads, dk, dv]} is added to
    each late GDN layer's filled recurrent state before the tail. Returns (logits of the last `keep` rows
    [keep, V] fp32, cache, P)."""
    n = int(ids.shape[0]) if hasattr(ids, "shape") else len(ids)
    if h_split.shape[0] != n:
        raise ValueError(f"h_split has {h_split.shape[0]} rows for {n} ids")
    if arm.fill == "swiftkv_native" or mix is not None:
        from ._lib import UnsupportedArchitecture
        raise UnsupportedArchitecture(f"arm {arm.name!r}: SwiftKV native and context arms are not implemented")
    _refuse_options(arm)
    P = arm.prefix_len(n)
    T = n - P
    if keep > T:
        raise ValueError(f"keep {keep} rows > exact tail {T}")
    split = arm.split
    dev = model.device
    h_split = h_split.to(dev, torch.bfloat16)
    cache = ([dict(c) for c in lower_cache[:split]] if lower_cache is not None else [dict() for _ in range(split)])
    cache += [dict() for _ in range(model.n_layers - split)]
    layers = list(range(split, model.n_layers))
    has_rows = exact_rows is not None and len(exact_rows) > 0
    if fill_reuse is not None and has_rows:
        raise ValueError("exact rows: sorted unique rows < P, no fill reuse")
    if P > 0 and fill_reuse is not None:
        for i in layers:
            got = fill_reuse[i].get("n", P)
            if got != P:
                raise ValueError(f"reused fill of layer {i} has {got} rows, P = {P}")
            cache[i] = dict(fill_reuse[i])
    for i in layers:                                 # a reused fill gets buffers of its own for its tail
        if model.layer_types[i] == "attn":
            model.reserve(cache[i], n - cache[i].get("n", 0), model.n_kv, model.head_dim, dev,
                          fresh=fill_reuse is not None and P > 0)
    if P > 0 and fill_reuse is None:
        fill_late(model, h_split, arm, exact_rows=exact_rows, hr=hr, cache=cache, row_inputs=row_inputs, oracle=oracle)
    if P > 0:
        for i in layers:
            if fill_store is not None:
                fill_store[i] = dict(cache[i])
            st = arm.st.get(i) if arm.st else None   # GDN terminal-state corrections (kva.py:452-454)
            if st is not None:
                if model.layer_types[i] != "gdn":
                    raise ValueError(f"st corrects GDN recurrent states; layer {i} is attention")
                cache[i]["rec"] = cache[i]["rec"] + st.to(cache[i]["rec"])
    h = h_split[P:]
    pos = torch.arange(P, n, device=dev)
    cs = model.rope_table(pos)
    ssq = ops.row_ssq(h)
    for i in layers:
        if hook is not None:
            hook(i, h)
        h, ssq = model.layer(i, h, pos, cache, ssq=ssq, cs=cs)
        if not keep_cache:
            cache[i] = {}
    return model.logits(h[T - keep:], ssq[T - keep:]), cache, P
