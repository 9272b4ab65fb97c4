"""Closed-form ridge maps on the GPU: RidgeStats / RidgeFit of code/kva/ridge.py with the sufficient
statistics accumulated by librfill's MFMA Gram kernel.

Per sample block (default 8192 rows, the reference's block): the block is transposed into the
K-contiguous operands X^T, Y_i^T (rf_transpose, which also yields the column sums), then
rf_gram_accumulate adds X^T X and X^T Y_i -- bf16 products summed in fp32 over the block, as the
reference's per-block fp32 GEMM (code/kva/ridge.py:47, :62) -- into fp64 accumulators. The device keeps
raw sums (n, sum x, X^T X, sum y_i, X^T Y_i); state() re-centres them in fp64 on the reference's shifts
(the first block's means, code/kva/ridge.py:37-38, :56-57), so the state dict has the reference's
layout and meaning. Shifting is exact algebra; what differs from shifting each block before its GEMM is
only the fp32 rounding inside a block, which grows with |mean| / spread of a channel.

RidgeFit solves W(lam) = (C + lam mean(diag C) I)^-1 Cxy with the bias unpenalised
(code/kva/ridge.py:80-105) in fp64 on the GPU by a Cholesky factorisation per lam (the same solution the
reference's eigendecomposition gives, since C + lam s I is symmetric positive definite for lam > 0).
"""
import torch

from . import _lib
from .ops import _need, _ptr, _stream


def _transpose(x, dst, partial):
    rows, cols = x.shape
    _lib.call("rf_transpose", _ptr(x), x.stride(0), rows, cols, _ptr(dst), dst.stride(0), _ptr(partial), _stream(x))


def _colsum_fold(partial, sums):
    _lib.call("rf_colsum_fold", _ptr(partial), partial.shape[0], partial.shape[1], _ptr(sums), _stream(sums))


def gram_accumulate(a, b, c):
    """c += a b^T (a [M, K], b [N, K] bf16 K-contiguous; c [M, N] fp64): fp32 over K, added in fp64."""
    _need(a, "a", torch.bfloat16, 2)
    _need(b, "b", torch.bfloat16, 2)
    _need(c, "c", torch.float64, 2)
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K or tuple(c.shape) != (M, N):
        raise ValueError(f"gram shapes a {tuple(a.shape)}, b {tuple(b.shape)}, c {tuple(c.shape)}")
    _lib.call("rf_gram_accumulate", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, _ptr(c), c.stride(0),
              _stream(a))
    return c


class RidgeStats:
    """Sufficient statistics of (x, y_i) pairs over every layer i, accumulated on the GPU."""

    def __init__(self, split, layers, dim, device="cuda", out_dim=None):
        self.split, self.layers, self.dim = split, list(layers), dim
        self.out_dim = dim if out_dim is None else out_dim
        self.device = torch.device(device)
        f64 = dict(dtype=torch.float64, device=self.device)
        self.n = 0
        self.cx, self.cy = None, {}
        self.s1x = torch.zeros(dim, **f64)
        self.sxx = torch.zeros(dim, dim, **f64)
        self.s1y = {i: torch.zeros(self.out_dim, **f64) for i in self.layers}
        self.sxy = {i: torch.zeros(dim, self.out_dim, **f64) for i in self.layers}

    @torch.no_grad()
    def add(self, x, ys, block=8192):
        """x [n, d] and ys {layer: [n, d_out]}: bf16 rows on the GPU (the same rows, in order)."""
        _need(x, "x", torch.bfloat16, 2)
        n, d = x.shape
        if d != self.dim or d % 256 or self.out_dim % 256:
            raise ValueError(f"x width {d} (stats dim {self.dim}); widths must be multiples of 256")
        if block % 64:
            raise ValueError("block must be a multiple of 64")
        if self.cx is None:
            self.cx = x[:block].float().mean(0)
        for i in self.layers:
            y = ys[i]
            _need(y, f"ys[{i}]", torch.bfloat16, 2)
            if tuple(y.shape) != (n, self.out_dim):
                raise ValueError(f"ys[{i}] shape {tuple(y.shape)}")
            if i not in self.cy:
                self.cy[i] = y[:block].float().mean(0)
        blk = min(block, (n + 63) // 64 * 64)
        xt = torch.empty(d, blk, dtype=torch.bfloat16, device=x.device)
        yt = torch.empty(self.out_dim, blk, dtype=torch.bfloat16, device=x.device)
        part = torch.empty(blk // 64, max(d, self.out_dim), dtype=torch.float32, device=x.device)
        for r in range(0, n, block):
            rows = min(block, n - r)
            kp = (rows + 63) // 64 * 64
            xt_b, yt_b = xt[:, :kp], yt[:, :kp]
            px = part[:kp // 64, :d]
            _transpose(x[r:r + rows], xt_b, px)
            _colsum_fold(px, self.s1x)
            gram_accumulate(xt_b, xt_b, self.sxx)
            for i in self.layers:
                py = part[:kp // 64, :self.out_dim]
                _transpose(ys[i][r:r + rows], yt_b, py)
                _colsum_fold(py, self.s1y[i])
                gram_accumulate(xt_b, yt_b, self.sxy[i])
        self.n += n

    def state(self, device="cpu"):
        """RidgeStats.state() (code/kva/ridge.py:70-74): shifted sums about cx / cy, fp64."""
        n = float(self.n)
        cx = self.cx.double()
        sx = self.s1x - n * cx
        sxx = self.sxx - torch.outer(cx, self.s1x) - torch.outer(self.s1x, cx) + n * torch.outer(cx, cx)
        cy, sy, sxy = {}, {}, {}
        for i in self.layers:
            c = self.cy[i].double()
            cy[i] = c.to(device)
            sy[i] = (self.s1y[i] - n * c).to(device)
            sxy[i] = (self.sxy[i] - torch.outer(cx, self.s1y[i]) - torch.outer(self.s1x, c) + n * torch.outer(cx, c)
                      ).to(device)
        return dict(split=self.split, layers=self.layers, dim=self.dim, n=self.n, cx=cx.to(device), cy=cy,
                    sx=sx.to(device), sxx=sxx.to(device), sy=sy, sxy=sxy)


class RidgeFit:
    """fp64 ridge solve on the GPU for every lambda (code/kva/ridge.py:77-105)."""

    def __init__(self, state, device="cuda"):
        dev = torch.device(device)
        self.state, self.device = state, dev
        n = state["n"]
        self.n = n
        sx = state["sx"].to(dev, torch.float64)
        self.sx = sx
        self.mean_x = state["cx"].to(dev, torch.float64) + sx / n
        self.cxx = state["sxx"].to(dev, torch.float64) - torch.outer(sx, sx) / n
        self.scale = self.cxx.diagonal().mean().item()
        self._chol = {}                                   # lam -> Cholesky factor, shared by every layer

    def cross(self, i):
        st = self.state
        sy = st["sy"][i].to(self.device, torch.float64)
        cxy = st["sxy"][i].to(self.device, torch.float64) - torch.outer(self.sx, sy) / self.n
        return cxy, st["cy"][i].to(self.device, torch.float64) + sy / self.n

    def solve(self, cxy, lam):
        if lam not in self._chol:
            a = self.cxx + (lam * self.scale) * torch.eye(self.cxx.shape[0], dtype=torch.float64, device=self.device)
            self._chol[lam] = torch.linalg.cholesky(a)
        return torch.cholesky_solve(cxy, self._chol[lam])

    def layer(self, i, lams):
        """{lam: (weight [d_out, d_in] fp32, bias [d_out] fp32)} for layer i (F.linear layout)."""
        return self.layers([i], lams)[i]

    def layers(self, ids, lams):
        """{i: {lam: (weight, bias)}} for every layer i in ids: the targets' cross statistics side by side,
        so each lambda costs one factorisation and one pair of triangular solves for all of them."""
        ids = list(ids)
        cross = [self.cross(i) for i in ids]
        cxy = torch.cat([c for c, _ in cross], 1)
        out = {i: {} for i in ids}
        for lam in lams:
            w_all = self.solve(cxy, lam)
            col = 0
            for i, (c, mean_y) in zip(ids, cross):
                w = w_all[:, col:col + c.shape[1]]
                col += c.shape[1]
                out[i][lam] = (w.T.float().contiguous(), (mean_y - self.mean_x @ w).float())
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
