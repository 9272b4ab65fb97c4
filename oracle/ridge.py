"""Oracle closed-form ridge (test infrastructure; see oracle/__init__.py).

Restates code/kva/ridge.py (RidgeStats :19-74, RidgeFit :77-105, residual :134-139, combine
:142-156) and the capture sums of code/scripts/fit_sweep.py (:62-166).

Sufficient statistics with fixed shifts c (the first block's / first document's means): n,
sx = sum(x - cx), sxx = (x - cx)^T (x - cx), sy_i = sum(y_i - cy_i), sxy_i = (x - cx)^T (y_i - cy_i);
fp32 products per block added into fp64. Fit (fp64): C = sxx - sx sx^T / n, scale = mean(diag C),
W(lam) = (C + lam scale I)^-1 Cxy with Cxy = sxy - sx sy^T / n, bias = mean_y - mean_x W (unpenalised);
returned as (W^T fp32 [d_out, d_in], bias fp32).
"""
import torch


class RidgeStats:
    """Per-block fp32 GEMMs into fp64 sums, shifts = the first block's means (code/kva/ridge.py:19-74)."""

    def __init__(self, split, layers, dim, out_dim=None):
        out_dim = dim if out_dim is None else out_dim
        self.split, self.layers, self.dim = split, list(layers), dim
        self.n = 0
        self.cx, self.cy = None, {}
        self.sx = torch.zeros(dim, dtype=torch.float64)
        self.sxx = torch.zeros(dim, dim, dtype=torch.float64)
        self.sy = {i: torch.zeros(out_dim, dtype=torch.float64) for i in self.layers}
        self.sxy = {i: torch.zeros(dim, out_dim, dtype=torch.float64) for i in self.layers}

    def add(self, x, ys, block=8192):
        if self.cx is None:
            self.cx = x[:block].float().mean(0)
        self.n += x.shape[0]
        for r in range(0, x.shape[0], block):
            xc = x[r:r + block].float() - self.cx
            self.sx += xc.sum(0).double()
            self.sxx += (xc.T @ xc).double()
        for i in self.layers:
            y = ys[i]
            if i not in self.cy:
                self.cy[i] = y[:block].float().mean(0)
            for r in range(0, y.shape[0], block):
                xc = x[r:r + block].float() - self.cx
                yc = y[r:r + block].float() - self.cy[i]
                self.sy[i] += yc.sum(0).double()
                self.sxy[i] += (xc.T @ yc).double()

    def state(self):
        return dict(split=self.split, layers=self.layers, dim=self.dim, n=self.n, cx=self.cx.double(),
                    cy={i: c.double() for i, c in self.cy.items()}, sx=self.sx, sxx=self.sxx,
                    sy=dict(self.sy), sxy=dict(self.sxy))


class Capture:
    """fit_sweep's capture sums over documents (code/scripts/fit_sweep.py:62-144): for every split S
    and late layer i >= S, shifts are the FIRST DOCUMENT's means (whole document, not a block)."""

    def __init__(self, splits, n_layers, dim):
        self.splits, self.L, self.dim = sorted(splits), n_layers, dim
        self.n = 0
        self.cx, self.cy = {}, {}
        self.sx = {S: torch.zeros(dim, dtype=torch.float64) for S in self.splits}
        self.sxx = {S: torch.zeros(dim, dim, dtype=torch.float64) for S in self.splits}
        pairs = [(S, i) for S in self.splits for i in range(S, n_layers)]
        self.sy = {p: torch.zeros(dim, dtype=torch.float64) for p in pairs}
        self.sxy = {p: torch.zeros(dim, dim, dtype=torch.float64) for p in pairs}

    def add_document(self, inputs):
        """inputs {layer: h [n_doc, dim]}: one document's layer inputs (every layer >= min split)."""
        xs = {}
        for i in sorted(inputs):
            h = inputs[i].float()
            if i in self.sx:
                if i not in self.cx:
                    self.cx[i] = h.mean(0)
                xs[i] = h - self.cx[i]
                self.sx[i] += xs[i].sum(0).double()
                self.sxx[i] += (xs[i].T @ xs[i]).double()
            for S in self.splits:
                if S <= i:
                    p = (S, i)
                    if p not in self.cy:
                        self.cy[p] = h.mean(0)
                    yc = h - self.cy[p]
                    self.sy[p] += yc.sum(0).double()
                    self.sxy[p] += (xs[S].T @ yc).double()
        self.n += next(iter(inputs.values())).shape[0]

    def state(self, S):
        late = list(range(S, self.L))
        return dict(split=S, layers=late, dim=self.dim, n=self.n, cx=self.cx[S].double(),
                    cy={i: self.cy[(S, i)].double() for i in late}, sx=self.sx[S], sxx=self.sxx[S],
                    sy={i: self.sy[(S, i)] for i in late}, sxy={i: self.sxy[(S, i)] for i in late})


class RidgeFit:
    """fp64 ridge for every lambda from one eigendecomposition of C (code/kva/ridge.py:77-105)."""

    def __init__(self, state):
        n = state["n"]
        self.n, self.state = n, state
        sx = state["sx"].double()
        self.mean_x = state["cx"].double() + sx / n
        cxx = state["sxx"].double() - torch.outer(sx, sx) / n
        self.cxx = cxx
        self.scale = cxx.diagonal().mean().item()
        self.evals, self.evecs = torch.linalg.eigh(cxx)

    def cross(self, i):
        st = self.state
        sx, sy = st["sx"].double(), st["sy"][i].double()
        cxy = st["sxy"][i].double() - torch.outer(sx, sy) / self.n
        return cxy, st["cy"][i].double() + sy / self.n

    def layer(self, i, lams):
        """{lam: (weight [d_out, d_in] fp32, bias [d_out] fp32)}."""
        cxy, mean_y = self.cross(i)
        a = self.evecs.T @ cxy
        out = {}
        for lam in lams:
            w = self.evecs @ (a / (self.evals + lam * self.scale)[:, None])
            out[lam] = (w.T.float().contiguous(), (mean_y - self.mean_x @ w).float())
        return out

    def layer_f64(self, i, lam):
        """The same solution in fp64 (the tolerance reference for an fp32 solve)."""
        cxy, mean_y = self.cross(i)
        w = self.evecs @ ((self.evecs.T @ cxy) / (self.evals + lam * self.scale)[:, None])
        return w.T.contiguous(), mean_y - self.mean_x @ w


def residual(state):
    """Statistics of the target y - x (code/kva/ridge.py:134-139)."""
    sx, sxx = state["sx"].double(), state["sxx"].double()
    L = state["layers"]
    return dict(state, sx=sx, sxx=sxx, cy={i: state["cy"][i] - state["cx"] for i in L},
                sy={i: state["sy"][i].double() - sx for i in L}, sxy={i: state["sxy"][i].double() - sxx for i in L})


def combine(a, b, w):
    """Statistics of a's rows plus w times b's rows, b re-centred on a's shifts (code/kva/ridge.py:142-156)."""
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
