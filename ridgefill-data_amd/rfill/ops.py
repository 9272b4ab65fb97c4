"""Torch-tensor front end of the librfill kernels (device memory and streams are PyTorch's; the
arithmetic is the HIP kernels'). Every function checks devices, dtypes and layouts before it hands
raw pointers to the C ABI, and launches on the current stream of the tensors' device."""
import ctypes
import math

import torch

from . import _lib
from ._lib import SSQ_COLS


def _stream(t):
    return ctypes_ptr(torch.cuda.current_stream(t.device).cuda_stream)


def ctypes_ptr(v):
    return v if v else None


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _need(t, name, dtype, dims=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be on a GPU (got {t.device}); the fill has no CPU path")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if dims is not None and t.dim() != dims:
        raise ValueError(f"{name}: {t.dim()}-d, expected {dims}-d")
    if t.dim() and t.stride(-1) != 1:
        raise ValueError(f"{name}: last dim must be contiguous")


def ssq_parts(h):
    """Partials per row for width h."""
    if h % SSQ_COLS:
        raise ValueError(f"hidden size {h} is not a multiple of {SSQ_COLS}")
    return h // SSQ_COLS


def gemm_workspace_bytes(M, N, K):
    """Bytes of the split-K workspace the GEMM entry points use for an M x N x K product (0: no split)."""
    b = ctypes.c_size_t(0)
    _lib.call("rf_gemm_workspace_bytes", M, N, K, ctypes.byref(b))
    return b.value


def rows_workspace_bytes(rows, N, K):
    """Bytes of the workspace norm_kv_rows / norm_qkv_rows require for `rows` scattered rows of an N x K
    product: they run 512 rows at a time, and a shorter last chunk may split K more ways than a full one."""
    b = ctypes.c_size_t(0)
    _lib.call("rf_rows_workspace_bytes", rows, N, K, ctypes.byref(b))
    return b.value


def _ws(workspace, M, N, K, device, need_of=None):
    """(pointer, bytes) of a GEMM's split-K workspace: None -> no split; "auto" -> allocated here when a
    split pays; a uint8 device tensor -> used if large enough. need_of: the size function (default
    gemm_workspace_bytes)."""
    if workspace is None:
        return None, 0
    if isinstance(workspace, str):
        need = (need_of or gemm_workspace_bytes)(M, N, K)
        if not need:
            return None, 0
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    _need(workspace, "workspace", torch.uint8, 1)
    return workspace, workspace.numel()


def map_apply(b, w, c, out=None, ssq=None, workspace=None):
    """x = b W^T + c in bf16 (Projector.__call__) and x's row sum-of-squares partials.
    b [P, h_in], w [h_out, h_in], c [h_out] or None. Returns (x [P, h_out], ssq [P, h_out / 256]).
    workspace: the split-K workspace (see _ws)."""
    _need(b, "b", torch.bfloat16, 2)
    _need(w, "w", torch.bfloat16, 2)
    if not w.is_contiguous():
        raise ValueError("w must be contiguous")
    if c is not None:
        _need(c, "c", torch.bfloat16, 1)
    P, h_in = b.shape
    h_out = w.shape[0]
    if w.shape[1] != h_in or (c is not None and c.shape[0] != h_out):
        raise ValueError(f"map shapes: b {tuple(b.shape)}, w {tuple(w.shape)}, c {None if c is None else tuple(c.shape)}")
    out = torch.empty(P, h_out, dtype=torch.bfloat16, device=b.device) if out is None else out
    ssq = torch.empty(P, ssq_parts(h_out), dtype=torch.float32, device=b.device) if ssq is None else ssq
    _need(out, "out", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    if tuple(out.shape) != (P, h_out) or tuple(ssq.shape) != (P, h_out // SSQ_COLS) or not ssq.is_contiguous():
        raise ValueError("map_apply: output shapes")
    ws, nb = _ws(workspace, P, h_out, h_in, b.device)
    _lib.call("rf_map_apply", _ptr(b), b.stride(0), _ptr(w), _ptr(c), _ptr(out), out.stride(0), _ptr(ssq),
              P, h_in, h_out, _ptr(ws), nb, _stream(b))
    return out, ssq


MAP_BATCH_MAX = 32        # layers per batched map / K-V launch (the library's per-layer pointer tables)


def _ptr_array(ts):
    """A host array of device pointers (NULL for None) for the batched entry points."""
    return (ctypes.c_void_p * len(ts))(*[_ptr(t) for t in ts])


def map_apply_batch(b, ws, cs, outs, ssqs):
    """Several late layers' maps in one launch (the fill loop of finish(), code/kva/kva.py:413-415, over
    every layer at once): outs[l] = b ws[l]^T + cs[l] and ssqs[l] its row sum-of-squares partials, each
    bit-identical to map_apply of that layer alone. Every layer reads the same rows b [P, h_in]; ws[l]
    [h_out, h_in], cs[l] [h_out] or None, outs[l] [P, h_out] (one row stride for all), ssqs[l]
    [P, h_out / 256] contiguous."""
    nl = len(ws)
    if not 0 < nl <= MAP_BATCH_MAX or not (len(cs) == len(outs) == len(ssqs) == nl):
        raise ValueError("map_apply_batch: one map, bias, output and statistics per layer")
    _need(b, "b", torch.bfloat16, 2)
    P, h_in = b.shape
    h_out = ws[0].shape[0]
    for i in range(nl):
        _need(ws[i], "w", torch.bfloat16, 2)
        _need(outs[i], "out", torch.bfloat16, 2)
        _need(ssqs[i], "ssq", torch.float32, 2)
        if tuple(ws[i].shape) != (h_out, h_in) or not ws[i].is_contiguous():
            raise ValueError(f"map_apply_batch: layer {i} map {tuple(ws[i].shape)}, expected ({h_out}, {h_in})")
        if cs[i] is not None:
            _need(cs[i], "c", torch.bfloat16, 1)
            if cs[i].shape[0] != h_out:
                raise ValueError(f"map_apply_batch: layer {i} bias width")
        if tuple(outs[i].shape) != (P, h_out) or outs[i].stride(0) != outs[0].stride(0):
            raise ValueError(f"map_apply_batch: layer {i} output {tuple(outs[i].shape)}, expected ({P}, {h_out})"
                             " with the row stride of layer 0's")
        if tuple(ssqs[i].shape) != (P, h_out // SSQ_COLS) or not ssqs[i].is_contiguous():
            raise ValueError(f"map_apply_batch: layer {i} statistics shape")
    _lib.call("rf_map_apply_batch", nl, _ptr(b), b.stride(0), _ptr_array(ws), _ptr_array(cs), _ptr_array(outs),
              outs[0].stride(0), _ptr_array(ssqs), P, h_in, h_out, _stream(b))


def norm_kv_write_batch(xs, ssqs, eps, wkvs, hkv, d, knorms, knorm_kind, cs, kbufs, vbufs, slot_begin):
    """The fused K / V fill (norm_kv_write) of several attention layers in one launch, each layer
    bit-identical to norm_kv_write of it alone: xs[l] [P, H] (one row stride), ssqs[l], wkvs[l]
    [2 hkv d, H], knorms[l] [d] (all given or all None), one RoPE table cs [P, rot] for every layer, and
    caches kbufs[l] / vbufs[l] [hkv, cap, d] of one shape and stride, rows [slot_begin, slot_begin + P)."""
    nl = len(xs)
    if not 0 < nl <= MAP_BATCH_MAX or not (len(ssqs) == len(wkvs) == len(knorms) == len(kbufs) == len(vbufs) == nl):
        raise ValueError("norm_kv_write_batch: one input, statistics, weights, k_norm and cache per layer")
    _need(cs, "cs", torch.bfloat16, 2)
    P, H = xs[0].shape
    hs, rs, cap = _cache_args(kbufs[0], vbufs[0], hkv, d, slot_begin, P)
    has_kn = knorms[0] is not None
    for i in range(nl):
        _need(xs[i], "x", torch.bfloat16, 2)
        _need(ssqs[i], "ssq", torch.float32, 2)
        _need(wkvs[i], "wkv", torch.bfloat16, 2)
        if tuple(xs[i].shape) != (P, H) or xs[i].stride(0) != xs[0].stride(0):
            raise ValueError(f"norm_kv_write_batch: layer {i} input {tuple(xs[i].shape)}, expected ({P}, {H}) with"
                             " layer 0's row stride")
        if tuple(ssqs[i].shape) != (P, ssq_parts(H)) or not ssqs[i].is_contiguous():
            raise ValueError(f"norm_kv_write_batch: layer {i} statistics shape")
        if tuple(wkvs[i].shape) != (2 * hkv * d, H) or not wkvs[i].is_contiguous():
            raise ValueError(f"norm_kv_write_batch: layer {i} wkv {tuple(wkvs[i].shape)}")
        if (knorms[i] is not None) != has_kn:
            raise ValueError("norm_kv_write_batch: k_norm gains for every layer or for none")
        if has_kn:
            _need(knorms[i], "knorm", torch.bfloat16, 1)
            if knorms[i].shape[0] != d:
                raise ValueError("norm_kv_write_batch: knorm width")
        if _cache_args(kbufs[i], vbufs[i], hkv, d, slot_begin, P) != (hs, rs, cap):
            raise ValueError(f"norm_kv_write_batch: layer {i} cache shape or strides differ from layer 0's")
    if cs.shape[0] != P or not cs.is_contiguous():
        raise ValueError("norm_kv_write_batch: cs rows")
    _lib.call("rf_norm_kv_write_batch", nl, _ptr_array(xs), xs[0].stride(0), _ptr_array(ssqs), P, H, float(eps),
              _ptr_array(wkvs), hkv, d, _ptr_array(knorms) if has_kn else None, int(knorm_kind), _ptr(cs),
              cs.shape[1], _ptr_array(kbufs), _ptr_array(vbufs), hs, rs, int(slot_begin), cap, _stream(xs[0]))


def norm_linear_batch(xs, ssqs, eps, ws, outs):
    """norm_linear of several entries in one launch (rf_norm_linear_batch): outs[l] = bf16(rms-normed xs[l] @
    ws[l]^T), each bit-identical to norm_linear of it alone without a workspace. Entry l: xs[l] [M_l, H] (one
    row stride for all), ssqs[l] [M_l, H / 256] contiguous, ws[l] [N_l, H] contiguous (N_l % 256 == 0),
    outs[l] [M_l, N_l] (one row stride for all)."""
    nl = len(xs)
    if not 0 < nl <= MAP_BATCH_MAX or not (len(ssqs) == len(ws) == len(outs) == nl):
        raise ValueError("norm_linear_batch: one input, statistics, weight and output per entry")
    H = xs[0].shape[1]
    rows, ns = [], []
    for i in range(nl):
        _need(xs[i], "x", torch.bfloat16, 2)
        _need(ssqs[i], "ssq", torch.float32, 2)
        _need(ws[i], "w", torch.bfloat16, 2)
        _need(outs[i], "out", torch.bfloat16, 2)
        M, N = xs[i].shape[0], ws[i].shape[0]
        if xs[i].shape[1] != H or xs[i].stride(0) != xs[0].stride(0):
            raise ValueError(f"norm_linear_batch: entry {i} input {tuple(xs[i].shape)}: width {H} and entry 0's row"
                             " stride expected")
        if tuple(ssqs[i].shape) != (M, ssq_parts(H)) or not ssqs[i].is_contiguous():
            raise ValueError(f"norm_linear_batch: entry {i} statistics shape")
        if tuple(ws[i].shape) != (N, H) or not ws[i].is_contiguous() or N % 256:
            raise ValueError(f"norm_linear_batch: entry {i} weight {tuple(ws[i].shape)}, expected (N % 256 == 0, {H})")
        if tuple(outs[i].shape) != (M, N) or outs[i].stride(0) != outs[0].stride(0) or outs[i].stride(1) != 1:
            raise ValueError(f"norm_linear_batch: entry {i} output {tuple(outs[i].shape)}, expected ({M}, {N})"
                             " with entry 0's row stride")
        rows.append(M)
        ns.append(N)
    _lib.call("rf_norm_linear_batch", nl, _ptr_array(xs), xs[0].stride(0), _ptr_array(ssqs),
              (ctypes.c_int64 * nl)(*rows), H, float(eps), _ptr_array(ws), (ctypes.c_int64 * nl)(*ns),
              _ptr_array(outs), outs[0].stride(0), _stream(xs[0]))


def row_ssq(x, ssq=None):
    """Row sum-of-squares partials [P, H / 256] of layer inputs x [P, H]."""
    _need(x, "x", torch.bfloat16, 2)
    P, H = x.shape
    ssq = torch.empty(P, ssq_parts(H), dtype=torch.float32, device=x.device) if ssq is None else ssq
    _need(ssq, "ssq", torch.float32, 2)
    if tuple(ssq.shape) != (P, H // SSQ_COLS) or not ssq.is_contiguous():
        raise ValueError("row_ssq: ssq shape")
    _lib.call("rf_row_ssq", _ptr(x), x.stride(0), _ptr(ssq), P, H, _stream(x))
    return ssq


def row_scatter(x, ssq, rows, hr):
    """In place: x[rows] = hr (bit-exact) and those rows' ssq partials (x.index_copy(0, rows, hr))."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(rows, "rows", torch.int64, 1)
    _need(hr, "hr", torch.bfloat16, 2)
    P, H = x.shape
    if hr.shape[1] != H or hr.shape[0] != rows.shape[0] or tuple(ssq.shape) != (P, ssq_parts(H)):
        raise ValueError("row_scatter: shapes")
    _lib.call("rf_row_scatter", _ptr(x), x.stride(0), _ptr(ssq), P, H, _ptr(rows), rows.shape[0], _ptr(hr),
              hr.stride(0), _stream(x))
    return x


def fold_norm(w, gain, kind):
    """bf16(w * gain) (kind 0, rms_norm) or bf16(w * (1 + gain)) (kind 1, rms_norm_zc), per column."""
    _need(w, "w", torch.bfloat16, 2)
    _need(gain, "gain", torch.bfloat16, 1)
    w = w.contiguous()
    gain = gain.contiguous()
    if gain.shape[0] != w.shape[1]:
        raise ValueError("fold_norm: gain width")
    out = torch.empty_like(w)
    _lib.call("rf_fold_norm", _ptr(w), _ptr(gain), int(kind), _ptr(out), w.shape[0], w.shape[1], _stream(w))
    return out


def rope_table(pos, inv_freq):
    """RoPE table [P, rot]: bf16 cos of the rot / 2 angles, then their bf16 sin (rope_cos_sin's half table)."""
    _need(pos, "pos", torch.int64, 1)
    _need(inv_freq, "inv_freq", torch.float32, 1)
    rot = 2 * inv_freq.shape[0]
    cs = torch.empty(pos.shape[0], rot, dtype=torch.bfloat16, device=pos.device)
    _lib.call("rf_rope_table", _ptr(pos.contiguous()), pos.shape[0], _ptr(inv_freq.contiguous()), rot, _ptr(cs),
              _stream(pos))
    return cs


def _cache_args(kbuf, vbuf, hkv, d, slot_begin, m):
    for name, t in (("kbuf", kbuf), ("vbuf", vbuf)):
        _need(t, name, torch.bfloat16, 3)
        if t.shape[0] != hkv or t.shape[2] != d:
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected [{hkv}, cap, {d}]")
    if kbuf.stride() != vbuf.stride() or kbuf.shape != vbuf.shape:
        raise ValueError("kbuf / vbuf must share shape and strides")
    return kbuf.stride(0), kbuf.stride(1), kbuf.shape[1]


def norm_kv_write(x, ssq, eps, wkv, hkv, d, knorm, knorm_kind, cs, kbuf, vbuf, slot_begin, workspace=None):
    """Fused fill of one attention layer: RMSNorm (gain folded into wkv), K / V projections, k_norm,
    RoPE, write of rows [slot_begin, slot_begin + P) into kbuf / vbuf [hkv, cap, d]."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(wkv, "wkv", torch.bfloat16, 2)
    _need(cs, "cs", torch.bfloat16, 2)
    P, H = x.shape
    if tuple(ssq.shape) != (P, ssq_parts(H)) or not ssq.is_contiguous():
        raise ValueError("norm_kv_write: ssq shape")
    if tuple(wkv.shape) != (2 * hkv * d, H) or not wkv.is_contiguous():
        raise ValueError(f"norm_kv_write: wkv {tuple(wkv.shape)}, expected ({2 * hkv * d}, {H})")
    if cs.shape[0] != P or not cs.is_contiguous():
        raise ValueError("norm_kv_write: cs rows")
    if knorm is not None:
        _need(knorm, "knorm", torch.bfloat16, 1)
        if knorm.shape[0] != d:
            raise ValueError("norm_kv_write: knorm width")
    hs, rs, cap = _cache_args(kbuf, vbuf, hkv, d, slot_begin, P)
    ws, nb = _ws(workspace, P, 2 * hkv * d, H, x.device)
    _lib.call("rf_norm_kv_write", _ptr(x), x.stride(0), _ptr(ssq), P, H, float(eps), _ptr(wkv), hkv, d,
              _ptr(knorm), int(knorm_kind), _ptr(cs), cs.shape[1], _ptr(kbuf), _ptr(vbuf), hs, rs,
              int(slot_begin), cap, _ptr(ws), nb, _stream(x))


def norm_kv_rows(x, ssq, eps, wkv, hkv, d, knorm, knorm_kind, cs, pos, kbuf, vbuf, workspace="auto", pos_max=None):
    """K / V of scattered rows x [rows, H] at positions pos (int64, device) into cache slots pos: the
    arithmetic of norm_kv_write, each row written to its own position's slot (the exact rows of a layer
    already filled from every prefix row). pos_max: a bound on pos known on the host (else read from the
    device, which waits for it); it must lie below the cache capacity and the table's rows. With pos_max
    given, the positions are not read back: the kernel skips any row whose position lies outside the cache
    or the table. workspace: "auto", or a uint8 tensor of at least rows_workspace_bytes bytes."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(wkv, "wkv", torch.bfloat16, 2)
    _need(cs, "cs", torch.bfloat16, 2)
    _need(pos, "pos", torch.int64, 1)
    rows, H = x.shape
    if tuple(ssq.shape) != (rows, ssq_parts(H)) or not ssq.is_contiguous():
        raise ValueError("norm_kv_rows: ssq shape")
    if tuple(wkv.shape) != (2 * hkv * d, H) or not wkv.is_contiguous():
        raise ValueError(f"norm_kv_rows: wkv {tuple(wkv.shape)}, expected ({2 * hkv * d}, {H})")
    if pos.shape[0] != rows or not pos.is_contiguous() or not cs.is_contiguous():
        raise ValueError("norm_kv_rows: pos / cs")
    if knorm is not None:
        _need(knorm, "knorm", torch.bfloat16, 1)
        if knorm.shape[0] != d:
            raise ValueError("norm_kv_rows: knorm width")
    hs, rs, cap = _cache_args(kbuf, vbuf, hkv, d, 0, rows)
    if rows == 0:
        return
    lim = min(cap, cs.shape[0])
    hi = int(pos.max().item()) if pos_max is None else int(pos_max)
    if pos_max is None and int(pos.min().item()) < 0:
        raise ValueError("norm_kv_rows: negative position")
    if hi >= lim:
        raise ValueError(f"norm_kv_rows: position {hi} beyond the cache ({cap} slots) or the table ({cs.shape[0]} rows)")
    ws, nb = _ws(workspace, rows, 2 * hkv * d, H, x.device, rows_workspace_bytes)
    _lib.call("rf_norm_kv_rows", _ptr(x), x.stride(0), _ptr(ssq), rows, H, float(eps), _ptr(wkv), hkv, d,
              _ptr(knorm), int(knorm_kind), _ptr(cs), cs.shape[1], _ptr(pos), lim, _ptr(kbuf), _ptr(vbuf), hs, rs,
              _ptr(ws), nb, _stream(x))


def norm_qkv_rows(x, ssq, eps, wqkv, hq, hkv, d, qnorm, knorm, norm_kind, cs, pos, kbuf, vbuf, out=None,
                  workspace="auto", pos_max=None):
    """norm_q and norm_kv_rows of the same rows from one product over wqkv = [wq; wkv]: returns the queries
    [rows, hq d] bf16 and writes the rows' K / V into cache slots pos (see norm_kv_rows for pos_max)."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(wqkv, "wqkv", torch.bfloat16, 2)
    _need(cs, "cs", torch.bfloat16, 2)
    _need(pos, "pos", torch.int64, 1)
    rows, H = x.shape
    if tuple(ssq.shape) != (rows, ssq_parts(H)) or not ssq.is_contiguous():
        raise ValueError("norm_qkv_rows: ssq shape")
    if tuple(wqkv.shape) != ((hq + 2 * hkv) * d, H) or not wqkv.is_contiguous():
        raise ValueError(f"norm_qkv_rows: wqkv {tuple(wqkv.shape)}, expected ({(hq + 2 * hkv) * d}, {H})")
    if pos.shape[0] != rows or not pos.is_contiguous() or not cs.is_contiguous():
        raise ValueError("norm_qkv_rows: pos / cs")
    for name, t in (("qnorm", qnorm), ("knorm", knorm)):
        if t is not None:
            _need(t, name, torch.bfloat16, 1)
            if t.shape[0] != d:
                raise ValueError(f"norm_qkv_rows: {name} width")
    hs, rs, cap = _cache_args(kbuf, vbuf, hkv, d, 0, rows)
    out = torch.empty(rows, hq * d, dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (rows, hq * d):
        raise ValueError("norm_qkv_rows: out shape")
    if rows == 0:
        return out
    lim = min(cap, cs.shape[0])
    hi = int(pos.max().item()) if pos_max is None else int(pos_max)
    if pos_max is None and int(pos.min().item()) < 0:
        raise ValueError("norm_qkv_rows: negative position")
    if hi >= lim:
        raise ValueError(f"norm_qkv_rows: position {hi} beyond the cache ({cap} slots) or the table ({cs.shape[0]} rows)")
    ws, nb = _ws(workspace, rows, (hq + 2 * hkv) * d, H, x.device, rows_workspace_bytes)
    _lib.call("rf_norm_qkv_rows", _ptr(x), x.stride(0), _ptr(ssq), rows, H, float(eps), _ptr(wqkv), hq, hkv, d,
              _ptr(qnorm), _ptr(knorm), int(norm_kind), _ptr(cs), cs.shape[1], _ptr(pos), lim, _ptr(out),
              out.stride(0), _ptr(kbuf), _ptr(vbuf), hs, rs, _ptr(ws), nb, _stream(x))
    return out


def rope_kv_write(k, v, cs, kbuf, vbuf, slot_begin):
    """fill_kv: RoPE on pre-RoPE k and the write of k / v [m, hkv, d] into rows [slot_begin, +m)."""
    for name, t in (("k", k), ("v", v)):
        _need(t, name, torch.bfloat16, 3)
        if t.stride(1) != t.shape[2]:
            raise ValueError(f"{name}: heads of one token must be contiguous")
    _need(cs, "cs", torch.bfloat16, 2)
    m, hkv, d = k.shape
    if tuple(v.shape) != (m, hkv, d) or cs.shape[0] != m or not cs.is_contiguous():
        raise ValueError("rope_kv_write: shapes")
    hs, rs, cap = _cache_args(kbuf, vbuf, hkv, d, slot_begin, m)
    _lib.call("rf_rope_kv_write", _ptr(k), k.stride(0), _ptr(v), v.stride(0), m, hkv, d, _ptr(cs), cs.shape[1],
              _ptr(kbuf), _ptr(vbuf), hs, rs, int(slot_begin), cap, _stream(k))


def norm_linear(x, ssq, eps, w, out=None, workspace=None):
    """bf16(rms-normed x @ w^T) with the norm gain already folded into w [N, H] (N % 256 == 0)."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(w, "w", torch.bfloat16, 2)
    P, H = x.shape
    N = w.shape[0]
    if w.shape[1] != H or not w.is_contiguous() or tuple(ssq.shape) != (P, ssq_parts(H)):
        raise ValueError("norm_linear: shapes")
    out = torch.empty(P, N, dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (P, N) or not ssq.is_contiguous():
        raise ValueError(f"norm_linear: out {tuple(out.shape)}, expected {(P, N)}; ssq must be contiguous")
    ws, nb = _ws(workspace, P, N, H, x.device)
    _lib.call("rf_norm_linear", _ptr(x), x.stride(0), _ptr(ssq), P, H, float(eps), _ptr(w), N, _ptr(out), out.stride(0),
              _ptr(ws), nb, _stream(x))
    return out


def row_gather(x, rows, out=None, ssq=None):
    """out = x[rows] (bit-exact) and its row sum-of-squares partials; rows int64 on the device."""
    _need(x, "x", torch.bfloat16, 2)
    _need(rows, "rows", torch.int64, 1)
    P, H = x.shape
    n = rows.shape[0]
    out = torch.empty(n, H, dtype=torch.bfloat16, device=x.device) if out is None else out
    ssq = torch.empty(n, ssq_parts(H), dtype=torch.float32, device=x.device) if ssq is None else ssq
    _need(out, "out", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    if tuple(out.shape) != (n, H) or tuple(ssq.shape) != (n, H // SSQ_COLS) or not ssq.is_contiguous():
        raise ValueError("row_gather: output shapes")
    _lib.call("rf_row_gather", _ptr(x), x.stride(0), P, H, _ptr(rows.contiguous()), n, _ptr(out), out.stride(0),
              _ptr(ssq), _stream(x))
    return out, ssq


def norm_q(x, ssq, eps, wq, hq, d, qnorm, qnorm_kind, cs, pos, out=None, workspace=None):
    """Queries of rows x at positions pos: RMSNorm (gain folded into wq), x wq^T, per-head q_norm, RoPE with
    table rows cs[pos]. Returns q [rows, hq d] bf16."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(wq, "wq", torch.bfloat16, 2)
    _need(cs, "cs", torch.bfloat16, 2)
    _need(pos, "pos", torch.int64, 1)
    rows, H = x.shape
    if tuple(wq.shape) != (hq * d, H) or not wq.is_contiguous() or tuple(ssq.shape) != (rows, ssq_parts(H)):
        raise ValueError(f"norm_q: wq {tuple(wq.shape)}, expected ({hq * d}, {H}); ssq {tuple(ssq.shape)}")
    if pos.shape[0] != rows or not cs.is_contiguous():
        raise ValueError("norm_q: pos / cs")
    if qnorm is not None:
        _need(qnorm, "qnorm", torch.bfloat16, 1)
    out = torch.empty(rows, hq * d, dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    ws, nb = _ws(workspace, rows, hq * d, H, x.device)
    _lib.call("rf_norm_q", _ptr(x), x.stride(0), _ptr(ssq), rows, H, float(eps), _ptr(wq), hq, d, _ptr(qnorm),
              int(qnorm_kind), _ptr(cs), cs.shape[1], _ptr(pos.contiguous()), _ptr(out), out.stride(0), _ptr(ws), nb,
              _stream(x))
    return out


def attend_rows_workspace_bytes(nq, hq, hkv, d, n):
    """Device bytes attend_rows uses to split the key range over more blocks (0: no split)."""
    b = ctypes.c_size_t(0)
    _lib.call("rf_attend_rows_workspace_bytes", nq, hq, hkv, d, n, ctypes.byref(b))
    return b.value


def attend_rows(q, qpos, kbuf, vbuf, n, hq, scale, out=None, workspace="auto"):
    """Causal attention of query rows q [nq, hq d] at sorted positions qpos over the first n cache rows of
    kbuf / vbuf [hkv, cap, d]. Returns [nq, hq d] bf16. workspace: uint8 device memory for the key-range
    splits ("auto": allocated here at the full size; None: no split)."""
    _need(q, "q", torch.bfloat16, 2)
    _need(qpos, "qpos", torch.int64, 1)
    for name, t in (("kbuf", kbuf), ("vbuf", vbuf)):
        _need(t, name, torch.bfloat16, 3)
    if kbuf.stride() != vbuf.stride() or kbuf.shape != vbuf.shape:
        raise ValueError("kbuf / vbuf must share shape and strides")
    hkv, cap, d = kbuf.shape
    nq = q.shape[0]
    if q.shape[1] < hq * d or qpos.shape[0] != nq or n > cap:
        raise ValueError("attend_rows: shapes")
    out = torch.empty(nq, hq * d, dtype=torch.bfloat16, device=q.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if isinstance(workspace, str):
        need = attend_rows_workspace_bytes(nq, hq, hkv, d, n)
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device) if need else None
    if workspace is not None:
        _need(workspace, "workspace", torch.uint8, 1)
    _lib.call("rf_attend_rows", _ptr(q), q.stride(0), _ptr(qpos.contiguous()), nq, hq, d, _ptr(kbuf), _ptr(vbuf), hkv,
              kbuf.stride(0), kbuf.stride(1), n, float(scale), _ptr(out), out.stride(0), _ptr(workspace),
              0 if workspace is None else workspace.numel(), _stream(q))
    return out


CAUSAL_GROUPS = (1, 2, 4, 8)            # query heads per K / V head rf_attend_causal takes at head_dim 64 / 128
CAUSAL_GROUPS_256 = (1, 2, 4, 8, 16)    # and at head_dim 256


def attend_causal_workspace_bytes(nq, hq, hkv, d, n):
    """Device bytes attend_causal uses for nq queries over n keys (the key-range splits' partials; may be 0)."""
    b = ctypes.c_size_t(0)
    _lib.call("rf_attend_causal_workspace_bytes", nq, hq, hkv, d, n, ctypes.byref(b))
    return b.value


def attend_causal(q, slot0, kbuf, vbuf, n, hq, scale, out=None, workspace=None, qpos=None):
    """Causal attention of queries q [nq, hq d] over the first n rows of kbuf / vbuf [hkv, cap, d]: query j
    sees keys 0 .. qpos[j] (qpos: sorted int64 positions on the device), or with qpos None the consecutive
    slots slot0 .. slot0 + nq - 1. Returns [nq, hq d] bf16. workspace: uint8 device memory of
    attend_causal_workspace_bytes (allocated here if None)."""
    _need(q, "q", torch.bfloat16, 2)
    for name, t in (("kbuf", kbuf), ("vbuf", vbuf)):
        _need(t, name, torch.bfloat16, 3)
    if kbuf.stride() != vbuf.stride() or kbuf.shape != vbuf.shape:
        raise ValueError("kbuf / vbuf must share shape and strides")
    hkv, cap, d = kbuf.shape
    nq = q.shape[0]
    if q.shape[1] < hq * d or n > cap:
        raise ValueError("attend_causal: shapes")
    if qpos is not None:
        _need(qpos, "qpos", torch.int64, 1)
        if qpos.shape[0] != nq:
            raise ValueError("attend_causal: one position per query")
        qpos = qpos.contiguous()
    out = torch.empty(nq, hq * d, dtype=torch.bfloat16, device=q.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if workspace is None:
        workspace = torch.empty(attend_causal_workspace_bytes(nq, hq, hkv, d, n), dtype=torch.uint8, device=q.device)
    _need(workspace, "workspace", torch.uint8, 1)
    if workspace.numel() == 0:
        workspace = None
    _lib.call("rf_attend_causal", _ptr(q), q.stride(0), nq, _ptr(qpos), int(slot0), hq, d, _ptr(kbuf), _ptr(vbuf),
              hkv, kbuf.stride(0), kbuf.stride(1), n, float(scale), _ptr(out), out.stride(0), _ptr(workspace),
              0 if workspace is None else workspace.numel(), _stream(q))
    return out


def residual_add(x, y, out=None, ssq=None):
    """out = bf16(x + y) and its row sum-of-squares partials."""
    _need(x, "x", torch.bfloat16, 2)
    _need(y, "y", torch.bfloat16, 2)
    rows, H = x.shape
    if tuple(y.shape) != (rows, H):
        raise ValueError("residual_add: shapes")
    out = torch.empty_like(x) if out is None else out
    ssq = torch.empty(rows, ssq_parts(H), dtype=torch.float32, device=x.device) if ssq is None else ssq
    _need(out, "out", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    if tuple(out.shape) != (rows, H) or tuple(ssq.shape) != (rows, H // SSQ_COLS) or not ssq.is_contiguous():
        raise ValueError(f"residual_add: out {tuple(out.shape)}, ssq {tuple(ssq.shape)} for rows {rows}, width {H}")
    _lib.call("rf_residual_add", _ptr(x), x.stride(0), _ptr(y), y.stride(0), _ptr(out), out.stride(0), _ptr(ssq), rows,
              H, _stream(x))
    return out, ssq


def map_apply_residual(x, w, res, out=None, ssq=None, workspace=None):
    """out = bf16(res + bf16(x w^T)) and its row sum-of-squares partials: map_apply without a bias then
    residual_add(res, .), bit-identical; with a few rows and a workspace the residual joins the split sums'
    epilogue."""
    _need(x, "x", torch.bfloat16, 2)
    _need(w, "w", torch.bfloat16, 2)
    _need(res, "res", torch.bfloat16, 2)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or not w.is_contiguous() or tuple(res.shape) != (M, N):
        raise ValueError(f"map_apply_residual: x {tuple(x.shape)}, w {tuple(w.shape)}, res {tuple(res.shape)}")
    out = torch.empty(M, N, dtype=torch.bfloat16, device=x.device) if out is None else out
    ssq = torch.empty(M, ssq_parts(N), dtype=torch.float32, device=x.device) if ssq is None else ssq
    _need(out, "out", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    if tuple(out.shape) != (M, N) or tuple(ssq.shape) != (M, N // SSQ_COLS) or not ssq.is_contiguous():
        raise ValueError("map_apply_residual: out / ssq shapes")
    ws, nb = _ws(workspace, M, N, K, x.device)
    _lib.call("rf_map_apply_residual", _ptr(x), x.stride(0), _ptr(w), _ptr(res), res.stride(0), _ptr(out),
              out.stride(0), _ptr(ssq), M, K, N, _ptr(ws), nb, _stream(x))
    return out, ssq


def norm_linear_swiglu(x, ssq, eps, w, out=None, workspace=None):
    """SwiGLU of the normed [gate; up] product: silu_mul(norm_linear(x, ssq, eps, w)) [rows, I],
    bit-identical; with a few rows and a workspace SwiGLU joins the split sums' epilogue."""
    _need(x, "x", torch.bfloat16, 2)
    _need(ssq, "ssq", torch.float32, 2)
    _need(w, "w", torch.bfloat16, 2)
    P, H = x.shape
    if w.shape[1] != H or w.shape[0] % 2 or not w.is_contiguous() or tuple(ssq.shape) != (P, ssq_parts(H)):
        raise ValueError(f"norm_linear_swiglu: x {tuple(x.shape)}, w {tuple(w.shape)}, ssq {tuple(ssq.shape)}")
    I = w.shape[0] // 2
    out = torch.empty(P, I, dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if out.shape[0] != P or out.shape[1] < I:
        raise ValueError(f"norm_linear_swiglu: out {tuple(out.shape)} for {P} rows of {I}")
    ws, nb = _ws(workspace, P, 2 * I, H, x.device)
    fused = ws is not None and P <= 512
    gu = None if fused else torch.empty(P, 2 * I, dtype=torch.bfloat16, device=x.device)
    _lib.call("rf_norm_linear_swiglu", _ptr(x), x.stride(0), _ptr(ssq), P, H, float(eps), _ptr(w), I, _ptr(out),
              out.stride(0), _ptr(gu), 0 if gu is None else gu.stride(0), _ptr(ws), nb, _stream(x))
    return out


def mfma_ceiling(blocks, iters, out):
    """rf_mfma_ceiling: blocks x 4 waves x 4 iters back-to-back bf16 MFMAs (32768 flop each) on register
    operands; out fp32 [blocks * 256] receives one value per thread. Time it to measure the MFMA throughput
    the power limit allows."""
    _need(out, "out", torch.float32, 1)
    if out.numel() < blocks * 256:
        raise ValueError(f"mfma_ceiling: out holds {out.numel()} values, needs {blocks * 256}")
    _lib.call("rf_mfma_ceiling", int(blocks), int(iters), _ptr(out), _stream(out))


def silu_mul(gu, out=None):
    """SwiGLU of gu = [gate | up] [rows, 2 I]: bf16(bf16(silu(gate)) * up) [rows, I]."""
    _need(gu, "gu", torch.bfloat16, 2)
    rows, two_i = gu.shape
    if two_i % 2:
        raise ValueError(f"silu_mul: gu width {two_i} is odd (expected gate and up halves)")
    I = two_i // 2
    out = torch.empty(rows, I, dtype=torch.bfloat16, device=gu.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (rows, I):
        raise ValueError(f"silu_mul: out {tuple(out.shape)}, expected {(rows, I)}")
    _lib.call("rf_silu_mul", _ptr(gu), gu.stride(0), rows, I, _ptr(out), out.stride(0), _stream(gu))
    return out


def gdn_workspace_bytes(rows, nk, nv, dk=128, dv=128):
    """Bytes of device workspace rf_gdn_fill needs to fill `rows` rows in one pass."""
    n = ctypes.c_size_t(0)
    _lib.call("rf_gdn_workspace_bytes", rows, nk, nv, dk, dv, ctypes.byref(n))
    return n.value


def _gdn_check(pre, nk, nv, dk, dv, conv_w, conv_in, a_log, dt_bias, state):
    _need(pre, "pre", torch.bfloat16, 2)
    _need(conv_w, "conv_w", torch.bfloat16, 2)
    _need(a_log, "a_log", torch.float32, 1)
    _need(dt_bias, "dt_bias", torch.float32, 1)
    _need(state, "state", torch.float32, 3)
    C = 2 * nk * dk + nv * dv
    if tuple(conv_w.shape) != (C, 4) or not conv_w.is_contiguous():
        raise ValueError(f"gdn_fill: conv weight {tuple(conv_w.shape)}, expected ({C}, 4)")
    if tuple(state.shape) != (nv, dk, dv) or not state.is_contiguous():
        raise ValueError(f"gdn_fill: state {tuple(state.shape)}")
    if pre.shape[1] < C + 2 * nv or a_log.numel() != nv or dt_bias.numel() != nv:
        raise ValueError(f"gdn_fill: rows {tuple(pre.shape)} (need >= {C + 2 * nv} columns), "
                         f"a_log {a_log.numel()}, dt_bias {dt_bias.numel()} (need {nv})")
    if conv_in is not None:
        _need(conv_in, "conv_in", torch.bfloat16, 2)
        if tuple(conv_in.shape) != (3, C) or not conv_in.is_contiguous():
            raise ValueError("gdn_fill: conv state shape")
    return C


def gdn_fill(pre, nk, nv, dk, dv, conv_w, conv_in, a_log, dt_bias, state, workspace=None):
    """Gated DeltaNet fill from in-projection rows pre [P, >= C + 2 nv] (q | k | v | b | a): updates
    state [nv, dk, dv] fp32 in place, returns the new conv state [3, C] bf16. workspace: uint8 device
    memory for the per-chunk products (None: allocated for one pass over P rows; a smaller one, of at
    least gdn_workspace_bytes(0, ...), makes several passes)."""
    C = _gdn_check(pre, nk, nv, dk, dv, conv_w, conv_in, a_log, dt_bias, state)
    if workspace is None:
        workspace = torch.empty(gdn_workspace_bytes(pre.shape[0], nk, nv, dk, dv), dtype=torch.uint8,
                                device=pre.device)
    _need(workspace, "workspace", torch.uint8, 1)
    conv_out = torch.empty(3, C, dtype=torch.bfloat16, device=pre.device)
    _lib.call("rf_gdn_fill", _ptr(pre), pre.stride(0), pre.shape[0], nk, nv, dk, dv, _ptr(conv_w), _ptr(conv_in),
              _ptr(conv_out), _ptr(a_log), _ptr(dt_bias), _ptr(state), _ptr(workspace), workspace.numel(),
              _stream(pre))
    return conv_out


class _GdnLayer(ctypes.Structure):
    _fields_ = [("pre", ctypes.c_void_p), ("ld", ctypes.c_int64), ("conv_w", ctypes.c_void_p),
                ("conv_in", ctypes.c_void_p), ("conv_out", ctypes.c_void_p), ("a_log", ctypes.c_void_p),
                ("dt_bias", ctypes.c_void_p), ("state", ctypes.c_void_p)]


GDN_BATCH_MAX = 2


def gdn_fill_batch(layers, nk, nv, dk, dv, workspace=None):
    """gdn_fill of up to GDN_BATCH_MAX independent layers over the same rows in one prep and one scan launch
    per pass: layers = [(pre, conv_w, conv_in, a_log, dt_bias, state)] (as gdn_fill's arguments; states updated
    in place). Returns their new conv states. Each is bit-identical to gdn_fill of that layer alone.
    workspace: split evenly between the layers (None: one pass each)."""
    n = len(layers)
    if not 1 <= n <= GDN_BATCH_MAX:
        raise ValueError(f"gdn_fill_batch: {n} layers (1 .. {GDN_BATCH_MAX})")
    P = layers[0][0].shape[0]
    arr = (_GdnLayer * n)()
    outs = []
    for j, (pre, conv_w, conv_in, a_log, dt_bias, state) in enumerate(layers):
        C = _gdn_check(pre, nk, nv, dk, dv, conv_w, conv_in, a_log, dt_bias, state)
        if pre.shape[0] != P:
            raise ValueError("gdn_fill_batch: every layer takes the same rows")
        conv_out = torch.empty(3, C, dtype=torch.bfloat16, device=pre.device)
        outs.append(conv_out)
        arr[j] = _GdnLayer(_ptr(pre), pre.stride(0), _ptr(conv_w), _ptr(conv_in), _ptr(conv_out), _ptr(a_log),
                           _ptr(dt_bias), _ptr(state))
    pre0 = layers[0][0]
    if workspace is None:
        workspace = torch.empty(n * gdn_workspace_bytes(P, nk, nv, dk, dv), dtype=torch.uint8, device=pre0.device)
    _need(workspace, "workspace", torch.uint8, 1)
    _lib.call("rf_gdn_fill_batch", arr, n, P, nk, nv, dk, dv, _ptr(workspace), workspace.numel(), _stream(pre0))
    return outs


def gdn_fill_noalloc(pre, nk, nv, dk, dv, conv_w, conv_in, a_log, dt_bias, state, conv_out=None):
    """gdn_fill through rf_gdn_fill_noalloc: the per-chunk workspace is the library's own device array, so
    the call allocates nothing beyond conv_out (pass one to allocate nothing at all). Bit-identical to
    gdn_fill. Calls that overlap on one GPU share that array: order them on one stream."""
    _need(pre, "pre", torch.bfloat16, 2)
    _need(conv_w, "conv_w", torch.bfloat16, 2)
    _need(a_log, "a_log", torch.float32, 1)
    _need(dt_bias, "dt_bias", torch.float32, 1)
    _need(state, "state", torch.float32, 3)
    C = 2 * nk * dk + nv * dv
    if tuple(conv_w.shape) != (C, 4) or not conv_w.is_contiguous() or tuple(state.shape) != (nv, dk, dv) \
            or not state.is_contiguous() or pre.shape[1] < C + 2 * nv or a_log.numel() != nv or dt_bias.numel() != nv:
        raise ValueError(f"gdn_fill_noalloc: pre {tuple(pre.shape)}, conv {tuple(conv_w.shape)}, "
                         f"state {tuple(state.shape)}")
    if conv_in is not None:
        _need(conv_in, "conv_in", torch.bfloat16, 2)
        if tuple(conv_in.shape) != (3, C) or not conv_in.is_contiguous():
            raise ValueError("gdn_fill_noalloc: conv state shape")
    if conv_out is None:
        conv_out = torch.empty(3, C, dtype=torch.bfloat16, device=pre.device)
    _need(conv_out, "conv_out", torch.bfloat16, 2)
    if tuple(conv_out.shape) != (3, C) or not conv_out.is_contiguous():
        raise ValueError("gdn_fill_noalloc: conv_out shape")
    _lib.call("rf_gdn_fill_noalloc", _ptr(pre), pre.stride(0), pre.shape[0], nk, nv, dk, dv, _ptr(conv_w),
              _ptr(conv_in), _ptr(conv_out), _ptr(a_log), _ptr(dt_bias), _ptr(state), _stream(pre))
    return conv_out


# ------------------------------------------------------------------------ exact-row selection

def gdn_forward_workspace_bytes(rows, nk, nv, dk=128, dv=128):
    """Bytes of device workspace rf_gdn_forward needs for `rows` rows in one pass."""
    n = ctypes.c_size_t(0)
    _lib.call("rf_gdn_forward_workspace_bytes", rows, nk, nv, dk, dv, ctypes.byref(n))
    return n.value


def gdn_forward(pre, nk, nv, dk, dv, conv_w, conv_in, a_log, dt_bias, state, out=None, workspace=None):
    """The exact GDN layer's mixing: as gdn_fill (state updated in place, returns the new conv state) and
    the delta-rule outputs [P, nv dv] bf16. Returns (out, conv state)."""
    _need(pre, "pre", torch.bfloat16, 2)
    _need(conv_w, "conv_w", torch.bfloat16, 2)
    _need(a_log, "a_log", torch.float32, 1)
    _need(dt_bias, "dt_bias", torch.float32, 1)
    _need(state, "state", torch.float32, 3)
    C = 2 * nk * dk + nv * dv
    if tuple(conv_w.shape) != (C, 4) or not conv_w.is_contiguous() or tuple(state.shape) != (nv, dk, dv) \
            or not state.is_contiguous() or pre.shape[1] < C + 2 * nv or a_log.numel() != nv or dt_bias.numel() != nv:
        raise ValueError(f"gdn_forward: pre {tuple(pre.shape)}, conv {tuple(conv_w.shape)}, state {tuple(state.shape)}")
    if conv_in is not None:
        _need(conv_in, "conv_in", torch.bfloat16, 2)
        if tuple(conv_in.shape) != (3, C) or not conv_in.is_contiguous():
            raise ValueError("gdn_forward: conv state shape")
    P = pre.shape[0]
    out = torch.empty(P, nv * dv, dtype=torch.bfloat16, device=pre.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    if out.shape[0] != P or out.shape[1] < nv * dv:
        raise ValueError(f"gdn_forward: out {tuple(out.shape)}")
    if workspace is None:
        workspace = torch.empty(gdn_forward_workspace_bytes(P, nk, nv, dk, dv), dtype=torch.uint8, device=pre.device)
    _need(workspace, "workspace", torch.uint8, 1)
    conv_out = torch.empty(3, C, dtype=torch.bfloat16, device=pre.device)
    _lib.call("rf_gdn_forward", _ptr(pre), pre.stride(0), P, nk, nv, dk, dv, _ptr(conv_w), _ptr(conv_in),
              _ptr(conv_out), _ptr(a_log), _ptr(dt_bias), _ptr(state), _ptr(out), out.stride(0), _ptr(workspace),
              workspace.numel(), _stream(pre))
    return out, conv_out


def sigmoid_mul(o, g, out=None):
    """bf16(o * bf16(sigmoid(g))) (Qwen3.5's attention output gate); out may be o."""
    _need(o, "o", torch.bfloat16, 2)
    _need(g, "g", torch.bfloat16, 2)
    rows, n = o.shape
    if tuple(g.shape) != (rows, n):
        raise ValueError(f"sigmoid_mul: o {tuple(o.shape)}, g {tuple(g.shape)}")
    out = torch.empty_like(o) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    _lib.call("rf_sigmoid_mul", _ptr(o), o.stride(0), _ptr(g), g.stride(0), rows, n, _ptr(out), out.stride(0),
              _stream(o))
    return out


def gated_rms_norm(x, z, weight, heads, dv, eps, out=None):
    """rms_norm_gated over [rows, heads dv]: bf16(bf16(weight * bf16(rms-normed x)) * silu(z))."""
    _need(x, "x", torch.bfloat16, 2)
    _need(z, "z", torch.bfloat16, 2)
    _need(weight, "weight", torch.bfloat16, 1)
    rows = x.shape[0]
    if z.shape[0] != rows or min(x.shape[1], z.shape[1]) < heads * dv or weight.numel() != dv:
        raise ValueError(f"gated_rms_norm: x {tuple(x.shape)}, z {tuple(z.shape)}, weight {weight.numel()}")
    out = torch.empty(rows, heads * dv, dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, 2)
    _lib.call("rf_gated_rms_norm", _ptr(x), x.stride(0), _ptr(z), z.stride(0), _ptr(weight), rows, heads, dv,
              float(eps), _ptr(out), out.stride(0), _stream(x))
    return out


def window_mass_workspace_bytes(w, hq, hkv, d, n_end):
    n = ctypes.c_size_t(0)
    _lib.call("rf_window_mass_workspace_bytes", w, hq, hkv, d, n_end, ctypes.byref(n))
    return n.value


def window_mass(q, pos0, kbuf, hq, scale, mass, workspace=None):
    """mass [>= pos0 + w] fp64 += the attention probability each key receives from the w window query
    rows q [w, >= hq d] (post-RoPE, at positions pos0 .. pos0 + w - 1) over the K cache kbuf [hkv, cap, d],
    summed over rows and query heads (code/kva/select.py:223-245, one layer)."""
    _need(q, "q", torch.bfloat16, 2)
    _need(kbuf, "kbuf", torch.bfloat16, 3)
    _need(mass, "mass", torch.float64, 1)
    hkv, cap, d = kbuf.shape
    w = q.shape[0]
    if q.shape[1] < hq * d or pos0 < 0 or pos0 + w > cap or mass.numel() < pos0 + w:
        raise ValueError(f"window_mass: q {tuple(q.shape)}, pos0 {pos0}, cache {tuple(kbuf.shape)}, "
                         f"mass {mass.numel()}")
    need = window_mass_workspace_bytes(w, hq, hkv, d, pos0 + w)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.call("rf_window_mass", _ptr(q), q.stride(0), w, pos0, hq, d, _ptr(kbuf), hkv, kbuf.stride(0),
              kbuf.stride(1), float(scale), _ptr(mass), _ptr(workspace), workspace.numel(), _stream(q))
    return mass


def read_cosine(pred, truth, na, nb, d, kgain, gain_kind, weight, out, workspace=None):
    """Read cosines of one layer and document (code/scripts/fit_sweep.py:307-313): each row of pred and truth
    [rows, >= (na + nb) d] bf16 holds na vectors of group a, then nb of group b, each d wide (an attention
    layer's K | V heads: na = nb = hkv; a GDN layer's q | k heads, its v heads or its [b | a] row, one call
    each on their column range). out[0] += weight * the sum of group a's cosines, group a's vectors scaled by
    the k_norm gain kgain [d] (or None) first; out[1] += weight * the sum of group b's when nb > 0."""
    _need(pred, "pred", torch.bfloat16, 2)
    _need(truth, "truth", torch.bfloat16, 2)
    _need(out, "out", torch.float64, 1)
    rows = pred.shape[0]
    if truth.shape[0] != rows or min(pred.shape[1], truth.shape[1]) < (na + nb) * d or out.numel() < (2 if nb else 1):
        raise ValueError(f"read_cosine: pred {tuple(pred.shape)}, truth {tuple(truth.shape)}, na {na}, nb {nb}, d {d}")
    if kgain is not None:
        _need(kgain, "kgain", torch.bfloat16, 1)
        if kgain.numel() != d:
            raise ValueError(f"read_cosine: kgain {kgain.numel()} values, vector width {d}")
    need = 8 * ((rows + 15) // 16)
    if workspace is None:
        workspace = torch.empty(max(need, 8), dtype=torch.uint8, device=pred.device)
    _lib.call("rf_read_cosine", _ptr(pred), pred.stride(0), _ptr(truth), truth.stride(0), rows, na, nb, d,
              _ptr(kgain), gain_kind, float(weight), _ptr(out), _ptr(workspace), workspace.numel(), _stream(pred))
    return out


# ------------------------------------------------------------------------ map formats

def dequant_i8_rows(codes, scale, group=128, out=None):
    """bf16 maps from int8 codes [rows, width] and their per-row group scales scale [rows, width / group]
    (bf16): out[i, j] = bf16(codes[i, j] * scale[i, j // group]), exact product, one rounding
    (the i8_row128 layout, code/c5/convert.py:91-97)."""
    _need(codes, "codes", torch.int8, 2)
    _need(scale, "scale", torch.bfloat16, 2)
    rows, width = codes.shape
    if group <= 0 or width % group or tuple(scale.shape) != (rows, width // group):
        raise ValueError(f"dequant_i8_rows: codes {tuple(codes.shape)}, scale {tuple(scale.shape)}, group {group}")
    if out is None:
        out = torch.empty(rows, width, dtype=torch.bfloat16, device=codes.device)
    _need(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (rows, width):
        raise ValueError(f"dequant_i8_rows: out {tuple(out.shape)}")
    _lib.call("rf_dequant_i8_rows", _ptr(codes), codes.stride(0), _ptr(scale), scale.stride(0), rows, width, group,
              _ptr(out), out.stride(0), _stream(codes))
    return out


GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


def dequant_gguf_rows(raw, ggml_type, width, out=None):
    """bf16 rows [rows, width] from the raw bytes raw [rows, >= row bytes] (uint8, on the device) of a
    GGUF tensor of ggml type F32, F16, Q8_0 (32-value blocks: fp16 scale, 32 int8 codes) or BF16; values
    exact in fp32, one round-to-nearest-even cast to bf16."""
    _need(raw, "raw", torch.uint8, 2)
    rows = raw.shape[0]
    if out is None:
        out = torch.empty(rows, width, dtype=torch.bfloat16, device=raw.device)
    _need(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (rows, width):
        raise ValueError(f"dequant_gguf_rows: out {tuple(out.shape)}, expected {(rows, width)}")
    _lib.call("rf_dequant_gguf_rows", int(ggml_type), _ptr(raw), raw.stride(0), rows, width, _ptr(out), out.stride(0),
              _stream(raw))
    return out


# ------------------------------------------------------------------------ host-side RoPE frequencies

def inv_freq_default(theta, rot_dim):
    """theta^(-2j/rot), fp32 on the host, as the reference computes it (code/kva/ops.py:42-43)."""
    return 1.0 / (theta ** (torch.arange(0, rot_dim, 2, dtype=torch.float32) / rot_dim))


def inv_freq_llama3(theta, dim, factor, low_freq_factor, high_freq_factor, original_max):
    """Llama-3.1 rescale of the default frequencies (code/kva/ops.py:46-56)."""
    inv = inv_freq_default(theta, dim)
    wavelen = 2 * math.pi / inv
    lo_wl, hi_wl = original_max / low_freq_factor, original_max / high_freq_factor
    scaled = torch.where(wavelen > lo_wl, inv / factor, inv)
    smooth = (original_max / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    mixed = (1 - smooth) * scaled / factor + smooth * scaled
    mid = (wavelen >= hi_wl) & (wavelen <= lo_wl)
    return torch.where(mid, mixed, scaled)
