"""Closed-form ridge maps on the GPU: RidgeStats / RidgeFit of code/kva/ridge.py with the sufficient
statistics accumulated by librfill's MFMA Gram kernel.

begin(x) / add_layer(i, y) (code/kva/ridge.py:34-62): up to PIECE rows at a time are transposed into the
K-contiguous operands X^T, Y_i^T (rf_transpose_centred, which also yields the column sums), then one
rf_gram_accumulate launch per operand pair adds X^T X or X^T Y_i: bf16 products summed in fp32 over runs of
at most `block` rows (default 8192, the reference's block), each run added into fp64 -- as the reference's
per-block fp32 GEMM (code/kva/ridge.py:47, :62) is. X^T is built once per piece and serves every layer.

Centring. The reference subtracts its shifts (the first block's means, code/kva/ridge.py:37-38, :56-57)
before each block's fp32 GEMM, which keeps the fp32 sums at the size of the centred values. Here the
channels whose first-block mean exceeds their spread (mean^2 > variance; at most SHIFT_MAX per operand,
largest ratio first) are centred in the transpose: their fp32 values x - shift go into the operand as three
bf16 rows whose sum is exact (hi in the main rows; mid and lo in the rows after them). One Gram product over
[main rows; mid and lo rows] then carries every centred product. The other channels, whose
raw sums are at most twice their centred size, are summed raw. state() combines the lo rows' products in
fp64 and moves every sum onto the reference's shifts by exact fp64 algebra, so the state dict has the
reference's layout and meaning.

RidgeFit solves W(lam) = (C + lam mean(diag C) I)^-1 Cxy with the bias unpenalised
(code/kva/ridge.py:80-105) in fp64 on the GPU with rf_ridge_solve: the inverse of C + lam s I by a block
recursion on its Schur complements, every product on fp64 MFMA, all lambdas and targets in each launch (the
same closed form the reference's eigendecomposition gives, since C + lam s I is symmetric positive definite
for lam > 0).
"""
import ctypes

import torch

from . import _lib
from .ops import _need, _ptr, _stream

SHIFT_MAX = 128      # channels per operand centred before the product (each takes a mid and a lo row)
LO_ROWS = 256        # extra rows per operand when any channel is centred (keeps the Gram width a multiple of 256)
PIECE = 65536        # rows transposed and multiplied per Gram launch
ROW_PAD = 64         # elements past the rows of a transposed operand: strides of 65536 or 8192 bf16 (a power of two)
                     # put all of a transpose block's output rows on the same memory channels (5 % slower)


def _transpose(x, dst, partial):
    rows, cols = x.shape
    _lib.call("rf_transpose", _ptr(x), x.stride(0), rows, cols, _ptr(dst), dst.stride(0), _ptr(partial), _stream(x))


def transpose_centred(x, dst, dst_lo, shift, lo_row, partial, partial_sq=None, n_centred=0):
    """x [rows, cols] bf16 -> dst [cols, >= round_up(rows, 64)]: values d = x - shift[c] (fp32) as bf16 hi, with
    the centred channels' exact remainder as bf16 mid in row lo_row[c] and lo in row n_centred + lo_row[c] of
    dst_lo (shift / lo_row / dst_lo None: a plain copy). partial / partial_sq: fp32 [tiles, cols] column sums /
    sums of squares of d per 64-row tile."""
    rows, cols = x.shape
    if (shift is None) != (lo_row is None) or (shift is not None and dst_lo is None):
        raise ValueError("transpose_centred: shift, lo_row and dst_lo go together")
    if shift is not None:
        _need(shift, "shift", torch.float32, 1)
        _need(lo_row, "lo_row", torch.int32, 1)
        if shift.numel() != cols or lo_row.numel() != cols or dst_lo.stride(0) != dst.stride(0) \
                or dst_lo.shape[0] < 2 * n_centred:
            raise ValueError("transpose_centred: shift / lo_row width, lo plane stride or rows")
    _lib.call("rf_transpose_centred", _ptr(x), x.stride(0), rows, cols, _ptr(shift), _ptr(lo_row), int(n_centred),
              _ptr(dst), dst.stride(0), _ptr(dst_lo), _ptr(partial), _ptr(partial_sq), _stream(x))


def tiles_view(buf, tiles, cols):
    """A dense [tiles, cols] fp32 view at the start of the flat buffer buf (the layout the transpose writes
    its per-tile column sums in and rf_colsum_fold reads)."""
    return buf.view(-1)[:tiles * cols].view(tiles, cols)


def _colsum_fold(partial, sums):
    _lib.call("rf_colsum_fold", _ptr(partial), partial.shape[0], partial.shape[1], _ptr(sums), _stream(sums))


def gram_workspace_bytes(M, N, K, fold_rows=0):
    """Bytes of rf_gram_accumulate's run-split workspace for this shape (0: it uses none)."""
    nb = ctypes.c_size_t(0)
    _lib.call("rf_gram_workspace_bytes", M, N, K, int(fold_rows), ctypes.byref(nb))
    return nb.value


def gram_upper_workspace_bytes(M, N, K, fold_rows=0):
    """Bytes of rf_gram_accumulate_upper's run-split workspace for this shape (0: it uses none)."""
    nb = ctypes.c_size_t(0)
    _lib.call("rf_gram_upper_workspace_bytes", M, N, K, int(fold_rows), ctypes.byref(nb))
    return nb.value


def gram_accumulate_upper(a, M, c, fold_rows=0, workspace=None):
    """The symmetric product c += a[:M] a^T (a [N, K] bf16 K-contiguous, M <= N; c [M, N] fp64), fp32 over runs
    of at most fold_rows of K, each run added in fp64 -- on c's block-upper 256 x 256 tiles only (tile column
    >= tile row), about half the work of gram_accumulate(a[:M], a, c); the block-lower tiles are left as they
    are (mirror_block_upper fills them). workspace as gram_accumulate's (gram_upper_workspace_bytes): at most
    one round of tiles all split into their runs, which keeps every CU busy. The block-upper tiles are
    bit-identical to gram_accumulate's."""
    _need(a, "a", torch.bfloat16, 2)
    _need(c, "c", torch.float64, 2)
    N, K = a.shape
    if not 0 <= M <= N or tuple(c.shape) != (M, N):
        raise ValueError(f"gram_upper shapes a {tuple(a.shape)}, M {M}, c {tuple(c.shape)}")
    need = gram_upper_workspace_bytes(M, N, K, fold_rows) if M > 0 and N % 256 == 0 and K % 64 == 0 else 0
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=c.device)
    nb = workspace.numel() if workspace is not None else 0
    _lib.call("rf_gram_accumulate_upper", _ptr(a), a.stride(0), M, N, K, int(fold_rows), _ptr(c), c.stride(0),
              _ptr(workspace), nb, _stream(a))
    return c


def mirror_block_upper(c):
    """c [M, N >= M]: the block-lower 256 x 256 tiles of c's leading M x M part (tile row > tile column) set
    from the block-upper ones (c[i, j] = c[j, i]), which gram_accumulate_upper accumulates."""
    M = c.shape[0]
    for r0 in range(256, M, 256):
        r1 = min(r0 + 256, M)
        c[r0:r1, :r0] = c[:r0, r0:r1].transpose(0, 1)
    return c


def gram_accumulate(a, b, c, fold_rows=0, workspace=None):
    """c += a b^T (a [M, K], b [N, K] bf16 K-contiguous; c [M, N] fp64): fp32 over runs of at most fold_rows
    of K (0: all of K), each run added in fp64. workspace: a uint8 device buffer for the run-split schedule
    of shapes just past one round of tiles (gram_workspace_bytes); taken from torch's allocator when None
    and needed. The result's bits do not depend on it."""
    _need(a, "a", torch.bfloat16, 2)
    _need(b, "b", torch.bfloat16, 2)
    _need(c, "c", torch.float64, 2)
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K or tuple(c.shape) != (M, N):
        raise ValueError(f"gram shapes a {tuple(a.shape)}, b {tuple(b.shape)}, c {tuple(c.shape)}")
    need = gram_workspace_bytes(M, N, K, fold_rows) if M > 0 and N % 256 == 0 and K % 64 == 0 else 0
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=c.device)
    nb = workspace.numel() if workspace is not None else 0
    _lib.call("rf_gram_accumulate", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, int(fold_rows), _ptr(c),
              c.stride(0), _ptr(workspace), nb, _stream(a))
    return c


class Centring:
    """One operand's centring: the reference's shift c [cols] (fp64 of an fp32 mean), the centred channels idx
    (sorted) with their shift (fp32, 0 elsewhere) and mid rows (int32, -1 elsewhere; the lo row is s rows
    further), and the number of extra rows the operand carries (0, or LO_ROWS when any channel is centred). Chosen from sums s1 / s2 of n rows: the
    shift is their mean unless c is given (a resumed state's shift); a channel is centred when its shift's
    square exceeds the rows' variance, largest ratio first, at most cap of them."""

    def __init__(self, s1, s2, n, c=None, cap=SHIFT_MAX):
        mean = s1 / n
        var = (s2 / n - mean * mean).clamp_min(0)
        self.c = mean.float().double() if c is None else c.to(s1.device, torch.float64)
        c2 = self.c * self.c
        big = (c2 > var).nonzero().flatten()
        ratio = c2[big] / var[big].clamp_min(1e-300)
        self.idx = big[ratio.argsort(descending=True, stable=True)[:cap]].sort().values
        cols = s1.numel()
        self.shift = torch.zeros(cols, dtype=torch.float32, device=s1.device)
        self.shift[self.idx] = self.c[self.idx].float()
        self.lo_row = torch.full((cols,), -1, dtype=torch.int32, device=s1.device)
        self.lo_row[self.idx] = torch.arange(self.idx.numel(), dtype=torch.int32, device=s1.device)
        self.s = int(self.idx.numel())
        self.lo_rows = LO_ROWS if self.s else 0
        self.delta = self.c - self.shift.double()       # the stored sums' shift -> the reference's shift

    @classmethod
    def of_rows(cls, x, work, part, part_sq, c=None, cap=SHIFT_MAX):
        """The centring chosen from rows x [n, cols] (their sums, via a plain transpose into work)."""
        n, cols = x.shape
        kp = (n + 63) // 64 * 64
        s1 = torch.zeros(cols, dtype=torch.float64, device=x.device)
        s2 = torch.zeros_like(s1)
        p1, p2 = tiles_view(part, kp // 64, cols), tiles_view(part_sq, kp // 64, cols)
        transpose_centred(x, work[:cols, :kp], None, None, None, p1, p2)
        _colsum_fold(p1, s1)
        _colsum_fold(p2, s2)
        return cls(s1, s2, n, c, cap)


def centred_products(G, ca, A, cb, B):
    """[ca, cb] fp64 sums of the operands' centred values d_a d_b from an augmented Gram G [ca + 2 A.s, >= cb +
    2 B.s]: rows (columns) ca .. ca + s - 1 are the mid parts and ca + s .. ca + 2 s - 1 the lo parts of the
    centred channels A.idx (B.idx); each centred channel's three parts are added in a fixed order."""
    def fold_cols(Gr):
        Dc = Gr[:, :cb].clone()
        if B.s:
            Dc[:, B.idx] += Gr[:, cb:cb + B.s]
            Dc[:, B.idx] += Gr[:, cb + B.s:cb + 2 * B.s]
        return Dc
    D = fold_cols(G[:ca])
    if A.s:
        D[A.idx] += fold_cols(G[ca:ca + A.s])
        D[A.idx] += fold_cols(G[ca + A.s:ca + 2 * A.s])
    return D


def recentre(D, s1a, s1b, da, db, n):
    """Sums about shifts moved by da / db: sum (d_a - da)(d_b - db)^T from D = sum d_a d_b^T, s1 = sum d.
    Updates D in place (the callers pass a fresh product) by three rank-1 updates: at d 4096 each term would
    otherwise be a 128 MB fp64 temporary."""
    D.addr_(da, s1b, alpha=-1.0)
    D.addr_(s1a, db, alpha=-1.0)
    D.addr_(da, db, alpha=float(n))
    return D


class RidgeStats:
    """Sufficient statistics of (x, y_i) pairs over every layer i, accumulated on the GPU. from_state()
    continues a saved state (the reference's resumable sufficient statistics, code/scripts/fit_sweep.py:20-25,
    :271-284)."""

    def __init__(self, split, layers, dim, device="cuda", out_dim=None, centre_max=SHIFT_MAX):
        """centre_max: at most this many channels per operand are centred before the product (0: raw sums
        re-centred in fp64 afterwards, which loses precision on channels whose mean dwarfs their spread)."""
        self.split, self.layers, self.dim = split, list(layers), dim
        self.centre_max = centre_max
        self.out_dim = dim if out_dim is None else out_dim
        self.device = torch.device(device)
        f64 = dict(dtype=torch.float64, device=self.device)
        self.n = 0
        self.cen_x, self.cen_y = None, {}
        self.s1x = torch.zeros(dim, **f64)
        self.s1y = {i: torch.zeros(self.out_dim, **f64) for i in self.layers}
        self.sxx, self.sxy = None, {}
        self.base = None
        self._x, self._xt = None, None

    @classmethod
    def from_state(cls, state, device="cuda"):
        """Statistics that continue `state` (a state() dict, e.g. saved and reloaded): new rows are summed about
        its shifts, and state() returns the saved and the new rows' statistics together."""
        dev = torch.device(device)
        L = list(state["layers"])
        out_dim = next(iter(state["sy"].values())).numel() if L else state["dim"]
        st = cls(state["split"], L, state["dim"], dev, out_dim)
        base = {k: state[k] for k in ("split", "layers", "dim", "n")}
        for k in ("cx", "sx", "sxx"):
            base[k] = state[k].to(dev, torch.float64)
        for k in ("cy", "sy", "sxy"):
            base[k] = {i: state[k][i].to(dev, torch.float64) for i in L}
        st.base = base
        return st

    def _buffers(self, kp):
        """Transposed-operand buffers for kp rows (grown as needed, kept between calls): X^T and Y^T with their
        extra rows, and the per-64-row column-sum partials."""
        if self._xt is None or self._xt.shape[1] - ROW_PAD < kp:
            d, o, lo = self.dim, self.out_dim, LO_ROWS
            self._xt = torch.zeros(d + lo, kp + ROW_PAD, dtype=torch.bfloat16, device=self.device)
            self._yt = torch.zeros(o + lo, kp + ROW_PAD, dtype=torch.bfloat16, device=self.device)
            self._part = torch.empty(kp // 64 * max(d, o), dtype=torch.float32, device=self.device)
            self._sq = torch.empty_like(self._part)
        return self._xt, self._yt, self._part

    def _gram(self, a, b, c, block):
        """gram_accumulate with a workspace kept between calls (grown as needed)."""
        need = gram_workspace_bytes(a.shape[0], b.shape[0], a.shape[1], block)
        gram_accumulate(a, b, c, block, self._workspace(need))

    def _gram_upper(self, a, M, c, block):
        """gram_accumulate_upper with the same kept workspace."""
        need = gram_upper_workspace_bytes(M, a.shape[0], a.shape[1], block)
        gram_accumulate_upper(a, M, c, block, self._workspace(need))

    def _workspace(self, need):
        ws = getattr(self, "_gws", None)
        if need and (ws is None or ws.numel() < need):
            self._gws = None                        # the old buffer goes before the larger one is taken
            self._gws = ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return ws

    def _x_piece(self, r, sums):
        """Rows r .. r + PIECE of the current boundary rows, centred and transposed into X^T (the column sums
        of their centred values added into s1x when `sums`); returns the row count."""
        x, d, cx = self._x, self.dim, self.cen_x
        rows = min(PIECE, x.shape[0] - r)
        kp = (rows + 63) // 64 * 64
        xt, _, part = self._buffers(kp)
        px = tiles_view(part, kp // 64, d)
        transpose_centred(x[r:r + rows], xt[:d, :kp], xt[d:, :kp], cx.shift, cx.lo_row, px, n_centred=cx.s)
        if sums:
            _colsum_fold(px, self.s1x)
        self._held = r
        return rows

    @torch.no_grad()
    def begin(self, x, block=8192, w=None):
        """Boundary rows x [n, d] (bf16, on the GPU) of one document: X^T X into the statistics. Follow with
        add_layer for every layer (code/kva/ridge.py:34-47). Rows go PIECE at a time through one Gram launch
        each, the fp32 sums running over at most `block` rows (the reference's block) before each is added
        into fp64. w (row weights) is not supported: the weighted fit is not part of the fill path."""
        if w is not None:
            raise NotImplementedError("RidgeStats.begin: row weights w are not supported on the device")
        _need(x, "x", torch.bfloat16, 2)
        n, d = x.shape
        if d != self.dim or d % 256 or self.out_dim % 256:
            raise ValueError(f"x width {d} (stats dim {self.dim}); widths must be multiples of 256")
        if block <= 0 or block % 64:
            raise ValueError("block must be a positive multiple of 64")
        self._x, self._block, self._held = x, block, None
        if n == 0:
            return
        if self.cen_x is None:                          # the first block's means are the shifts (ridge.py:37-38)
            kp = (min(block, n) + 63) // 64 * 64
            xt, _, part = self._buffers(kp)
            b = self.base
            self.cen_x = Centring.of_rows(x[:block], xt, part, self._sq, None if b is None else b["cx"],
                                          self.centre_max)
            self.sxx = torch.zeros(d + 2 * self.cen_x.s, d + self.cen_x.lo_rows, dtype=torch.float64,
                                   device=self.device)
        cx = self.cen_x
        self.n += n
        for r in range(0, n, PIECE):
            rows = self._x_piece(r, True)
            kp = (rows + 63) // 64 * 64
            xt = self._xt
            self._gram_upper(xt[:d + cx.lo_rows, :kp], d + 2 * cx.s, self.sxx, block)
            self._sxx_upper = True

    @torch.no_grad()
    def add_layer(self, i, y):
        """The same rows' true inputs y [n, d_out] of layer i (code/kva/ridge.py:54-62): X^T Y_i into the statistics."""
        if i not in self.s1y:
            raise KeyError(f"layer {i} is not one of the statistics' layers {self.layers}")
        x = getattr(self, "_x", None)
        if x is None:
            raise ValueError("add_layer before begin")
        _need(y, f"y[{i}]", torch.bfloat16, 2)
        n = x.shape[0]
        if tuple(y.shape) != (n, self.out_dim):
            raise ValueError(f"y[{i}] shape {tuple(y.shape)}; want ({n}, {self.out_dim})")
        if n == 0:
            return
        d, o, block, cx = self.dim, self.out_dim, self._block, self.cen_x
        if i not in self.cen_y:
            kp = (min(block, n) + 63) // 64 * 64
            _, yt, part = self._buffers(kp)
            b = self.base
            self.cen_y[i] = Centring.of_rows(y[:block], yt, part, self._sq, None if b is None else b["cy"][i],
                                             self.centre_max)
        cy = self.cen_y[i]
        if i not in self.sxy:
            self.sxy[i] = torch.zeros(d + 2 * cx.s, o + cy.lo_rows, dtype=torch.float64, device=self.device)
        for r in range(0, n, PIECE):
            rows = self._x_piece(r, False) if self._held != r else min(PIECE, n - r)
            kp = (rows + 63) // 64 * 64
            xt, yt, part = self._buffers(kp)
            py = tiles_view(part, kp // 64, o)
            transpose_centred(y[r:r + rows], yt[:o, :kp], yt[o:, :kp], cy.shift, cy.lo_row, py, n_centred=cy.s)
            _colsum_fold(py, self.s1y[i])
            self._gram(xt[:d + 2 * cx.s, :kp], yt[:o + cy.lo_rows, :kp], self.sxy[i], block)

    def add(self, x, ys, block=8192, w=None):
        """x [n, d] and ys {layer: [n, d_out]}: bf16 rows on the GPU (the same rows, in order)
        (code/kva/ridge.py:64-68)."""
        self.begin(x, block, w)
        for i in self.layers:
            self.add_layer(i, ys[i])

    def state(self, device="cpu"):
        """RidgeStats.state() (code/kva/ridge.py:70-74): shifted sums about cx / cy, fp64."""
        if self.cen_x is None:
            if self.base is None:
                raise ValueError("no rows added")
            return _to(self.base, device)
        n = float(self.n)
        d, o, cx = self.dim, self.out_dim, self.cen_x
        dx = cx.delta
        if getattr(self, "_sxx_upper", False):      # X^T X accumulated on its block-upper tiles only
            mirror_block_upper(self.sxx)
        sxx = recentre(centred_products(self.sxx, d, cx, d, cx), self.s1x, self.s1x, dx, dx, n)
        cy, sy, sxy = {}, {}, {}
        for i in self.layers:
            if i not in self.cen_y:                 # no rows of this layer yet: zero sums, no shift (ridge.py:73)
                sy[i] = self.s1y[i].clone()
                sxy[i] = torch.zeros(d, o, dtype=torch.float64, device=self.device)
                if self.base is not None:           # resumed: zero sums about the saved shift, so combine()
                    cy[i] = self.base["cy"][i]      # carries the saved sums of this layer unchanged
                continue
            c = self.cen_y[i]
            cy[i] = c.c
            sy[i] = self.s1y[i] - n * c.delta
            sxy[i] = recentre(centred_products(self.sxy[i], d, cx, o, c), self.s1x, self.s1y[i], dx, c.delta, n)
        mine = dict(split=self.split, layers=self.layers, dim=self.dim, n=self.n, cx=cx.c, cy=cy,
                    sx=self.s1x - n * dx, sxx=sxx, sy=sy, sxy=sxy)
        return _to(combine(self.base, mine, 1) if self.base is not None else mine, device)


def _to(state, device):
    out = {}
    for k, v in state.items():
        if isinstance(v, torch.Tensor):
            out[k] = v.to(device)
        elif isinstance(v, dict):
            out[k] = {i: t.to(device) if isinstance(t, torch.Tensor) else t for i, t in v.items()}
        else:
            out[k] = v
    return out


def ridge_solve_workspace_bytes(d, nlam=1):
    n = ctypes.c_size_t(0)
    _lib.call("rf_ridge_solve_workspace_bytes", d, nlam, ctypes.byref(n))
    return n.value


class RidgeFit:
    """fp64 ridge solve on the GPU for every lambda (code/kva/ridge.py:77-105): rf_ridge_solve inverts
    C + lam mean(diag C) I (block recursion on Schur complements, fp64 MFMA products) and multiplies the
    cross statistics of every target at once; the bias is unpenalised (mean_y - mean_x W)."""

    def __init__(self, state, device="cuda"):
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError("RidgeFit solves on the GPU (rf_ridge_solve); device must be a GPU")
        self.state, self.device = state, dev
        n = state["n"]
        self.n = n
        sx = state["sx"].to(dev, torch.float64)
        self.sx = sx
        self.mean_x = state["cx"].to(dev, torch.float64) + sx / n
        self.cxx = torch.addr(state["sxx"].to(dev, torch.float64), sx, sx, alpha=-1.0 / n).contiguous()
        self.scale = self.cxx.diagonal().mean().item()

    def cross(self, i, out=None):
        """(cross statistics [d, d_out] of target i about the means, mean_y [d_out]); out: where to write the
        former (e.g. the target's columns of the side-by-side matrix the solve takes)."""
        st = self.state
        sy = st["sy"][i].to(self.device, torch.float64)
        sxy = st["sxy"][i].to(self.device, torch.float64)
        cxy = torch.addr(sxy, self.sx, sy, alpha=-1.0 / self.n, out=out)
        return cxy, st["cy"][i].to(self.device, torch.float64) + sy / self.n

    def solve(self, cxy, lams, mean_y=None):
        """(W [nlam, d, R], bias [nlam, R] or None) fp64: (C + lam s I)^-1 cxy for each lam, and mean_y - mean_x W."""
        lams = [float(v) for v in lams]
        cxy = cxy.to(self.device, torch.float64).contiguous()
        d, R = cxy.shape
        if d % 2 or R % 2:
            raise ValueError(f"ridge solve: d {d} and R {R} must be even")
        f64 = dict(dtype=torch.float64, device=self.device)
        w = torch.empty(len(lams), d, R, **f64)
        bias = None if mean_y is None else torch.empty(len(lams), R, **f64)
        ws = torch.empty(ridge_solve_workspace_bytes(d, len(lams)), dtype=torch.uint8, device=self.device)
        arr = (ctypes.c_double * len(lams))(*lams)
        mx = self.mean_x.contiguous()
        my = None if mean_y is None else mean_y.to(self.device, torch.float64).contiguous()
        _lib.call("rf_ridge_solve", _ptr(self.cxx), self.cxx.stride(0), d, _ptr(cxy), cxy.stride(0), R,
                  _ptr(mx) if my is not None else None, _ptr(my), arr, len(lams), float(self.scale), _ptr(w), R, d * R,
                  _ptr(bias), R, _ptr(ws), ws.numel(), _stream(cxy))
        return w, bias

    def layer(self, i, lams):
        """{lam: (weight [d_out, d_in] fp32, bias [d_out] fp32)} for layer i (F.linear layout)."""
        return self.layers([i], lams)[i]

    def layers(self, ids, lams):
        """{i: {lam: (weight, bias)}} for every layer i in ids: the targets' cross statistics side by side,
        one rf_ridge_solve for every lambda and target."""
        ids, lams = list(ids), list(lams)
        widths = [self.state["sxy"][i].shape[1] for i in ids]
        cols = [0]
        for k in widths:
            cols.append(cols[-1] + k)
        cxy = torch.empty(self.cxx.shape[0], cols[-1], dtype=torch.float64, device=self.device)
        means = [self.cross(i, out=cxy[:, cols[j]:cols[j + 1]])[1] for j, i in enumerate(ids)]
        w_all, b_all = self.solve(cxy, lams, torch.cat(means))
        del cxy
        out = {i: {} for i in ids}
        for j, i in enumerate(ids):             # one transposing fp32 copy per target for all lambdas
            c0, c1 = cols[j], cols[j + 1]
            wt = w_all[:, :, c0:c1].transpose(1, 2).to(torch.float32, memory_format=torch.contiguous_format)
            bt = b_all[:, c0:c1].float()
            for li, lam in enumerate(lams):
                out[i][lam] = (wt[li], bt[li])
        return out


def residual(state):
    """Statistics of the target y - x (code/kva/ridge.py:134-139)."""
    sx, sxx = state["sx"].double(), state["sxx"].double()
    L = state["layers"]
    return dict(state, sx=sx, sxx=sxx, cy={i: state["cy"][i] - state["cx"] for i in L},
                sy={i: state["sy"][i].double() - sx for i in L}, sxy={i: state["sxy"][i].double() - sxx for i in L})


def combine(a, b, w):
    """Statistics of a's rows plus w times b's rows about a's shifts (code/kva/ridge.py:142-156)."""
    d = b["cx"] - a["cx"]
    nb = b["n"]
    out = dict(a, n=a["n"] + w * nb)
    out["sx"] = a["sx"] + w * (b["sx"] + nb * d)
    out["sxx"] = a["sxx"] + w * (b["sxx"] + torch.outer(b["sx"], d) + torch.outer(d, b["sx"]) + nb * torch.outer(d, d))
    out["sy"], out["sxy"] = {}, {}
    for i in a["layers"]:
        e = b["cy"][i] - a["cy"][i]
        out["sy"][i] = a["sy"][i] + w * (b["sy"][i] + nb * e)
        out["sxy"][i] = a["sxy"][i] + w * (b["sxy"][i] + torch.outer(b["sx"], e) + torch.outer(d, b["sy"][i])
                                           + nb * torch.outer(d, e))
    return out
