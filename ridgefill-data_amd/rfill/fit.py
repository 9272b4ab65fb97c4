"""The fit driver on the GPU: the capture pass, the per-split ridge fit and the held-out lambda selection
of code/scripts/fit_sweep.py, over FillModel's exact forward and librfill's kernels.

Capture (fit_sweep.py:62-166, :236-248). One exact forward per calibration document
(FillModel.forward_exact, stopped before the last layer, whose output no split needs). The inputs h_i of
every layer i >= the smallest split S0 are transposed (rf_transpose) into one K-contiguous block
T [(L - S0) H, B] bf16: layer i owns rows (i - S0) H .. + H, documents sit side by side at 64-row
offsets, and the padding columns are zero, so they add nothing to any sum. When the block is full (or a
state is asked for), one rf_gram_accumulate per split S adds T_S [H, K] times T_{S..L-1}^T into that
split's fp64 accumulator [H, (L - S) H]: its first H columns are X_S^T X_S and its column block i - S is
X_S^T H_i -- every (S, i) pair of the reference in one MFMA launch per split, over up to B rows at a time.
The column sums of each layer come from the transpose (rf_colsum_fold) and serve every split.

Centring, as in rfill.ridge: the reference subtracts its shifts -- the first document's means of h_S and of
h_i (fit_sweep.py:98-99, :104-105) -- before its per-document fp32 GEMM. Here each layer's channels whose
first-document mean exceeds their spread (at most ridge.SHIFT_MAX) are centred in the transpose, as three
bf16 parts whose sum is exact; every layer owns H main rows and ridge.LO_ROWS extra rows of the block, and
the extra rows' products come out of the same Gram launch. state(S) combines them in fp64 and moves every sum onto the
reference's shifts (the first document's fp64 column sums over its row count, rounded to fp32 as the
reference's h.float().mean(0) is), so the state dict has split_state()'s layout and meaning
(fit_sweep.py:147-166). Products are bf16 x bf16 (exact) summed in fp32 over a block on MFMA and added
into fp64, as the reference's per-document fp32 GEMM is added into fp64.

Selection (fit_sweep.py:298-318). For each held-out document: one exact forward (stopped after the last
layer's input); per late layer i the true reads, one norm_linear GEMM: norm(h_i) [W_k; W_v]^T for an
attention layer (the pre-RoPE K | V of code/kva/model.py:282-287), norm(h_i) [W_qkv; W_b; W_a]^T for a
GDN layer (its pre-conv q | k | v and [b | a], code/kva/model.py:566-571); per candidate (each lambda's
map, then the identity) the predicted input x = h_S W^T + b (rf_map_apply) and its reads; rf_read_cosine
adds the document's mean cosine of each read (K and V, k_norm gain applied for Qwen3 / Qwen3.5; or q, k, v
and [b | a]) into an fp64 score per candidate and layer, which averages them.
"""
import torch

from . import ops, ridge
from ._lib import UnsupportedArchitecture
from .kva import Projector

LAMBDAS = (1e-4, 3e-4, 1e-3, 3e-3, 0.01, 0.03, 0.1, 0.3, 1.0)      # fit_sweep.py:44
BLOCK = 8192


class Capture:
    """fit_sweep's capture sums for every split in splits over the documents added (add_document)."""

    def __init__(self, model, splits, block=BLOCK):
        self.model, self.splits = model, sorted(set(int(s) for s in splits))
        self.L, H = model.n_layers, model.hidden
        if not self.splits or self.splits[0] < 1 or self.splits[-1] >= self.L:
            raise ValueError(f"splits {splits}: each split S needs 1 <= S < {self.L} (late layers S .. L - 1)")
        if H % 256:
            raise ValueError(f"hidden size {H}: the Gram accumulation needs a multiple of 256")
        if block <= 0 or block % 64:
            raise ValueError("block must be a positive multiple of 64")
        self.S0, self.H, self.block = self.splits[0], H, block
        self.R = H + ridge.LO_ROWS                        # block rows per layer: H main rows, then the lo rows
        dev = model.device
        f64 = dict(dtype=torch.float64, device=dev)
        nl = self.L - self.S0
        self.n, self.docs = 0, 0
        self.s1 = torch.zeros(nl, H, **f64)               # column sums of each layer's centred values
        self.cen = [None] * nl                            # each layer's centring (from the first document)
        self.acc = {S: torch.zeros(self.R, (self.L - S) * self.R, **f64) for S in self.splits}
        self.T = None
        self.part = self.part_sq = None
        self.off = 0

    def _room(self, kp):
        cap = self.T.shape[1] - ridge.ROW_PAD if self.T is not None else 0
        if kp > cap:
            self.flush()
            cap = max(self.block, kp)
            dev = self.model.device
            self.T = torch.zeros((self.L - self.S0) * self.R, cap + ridge.ROW_PAD, dtype=torch.bfloat16, device=dev)
            self.part = torch.empty(cap // 64, self.H, dtype=torch.float32, device=dev)
            self.part_sq = torch.empty_like(self.part)
        elif self.off + kp > cap:
            self.flush()

    def _hook(self, i, h):
        if i == "final" or i < self.S0:
            return
        j = i - self.S0
        kp = (h.shape[0] + 63) // 64 * 64
        r = j * self.R
        main, lo = self.T[r:r + self.H, self.off:self.off + kp], self.T[r + self.H:r + self.R, self.off:self.off + kp]
        part = ridge.tiles_view(self.part, kp // 64, self.H)
        if self.cen[j] is None:                           # the first document: its means are the shifts
            self.cen[j] = ridge.Centring.of_rows(h, self.T[r:r + self.H, self.off:], self.part, self.part_sq)
        c = self.cen[j]
        ridge.transpose_centred(h, main, lo, c.shift, c.lo_row, part, n_centred=c.s)
        ridge._colsum_fold(part, self.s1[j])

    @torch.no_grad()
    def add_document(self, ids):
        """One calibration document's token ids: its exact forward, every layer input >= S0 into the sums."""
        n = int(torch.as_tensor(ids).numel())
        if n == 0:
            raise ValueError("empty document")
        kp = (n + 63) // 64 * 64
        self._room(kp)
        self.model.forward_exact(ids, hook=self._hook, stop=self.L - 1)
        self.off += kp
        self.docs += 1
        self.n += n

    def flush(self):
        """Add the buffered rows' products into every split's accumulator."""
        if not self.off:
            return
        K, H, R = self.off, self.H, self.R
        for S in self.splits:
            r = (S - self.S0) * R
            m = H + 2 * self.cen[S - self.S0].s
            ridge.gram_accumulate(self.T[r:r + m, :K], self.T[r:, :K], self.acc[S][:m], self.block)
        self.off = 0

    def state(self, S, device="cpu"):
        """split_state(acc, S, L, H) (fit_sweep.py:147-166): fp64 sums about the first document's means."""
        if S not in self.acc:
            raise KeyError(f"split {S} was not captured (splits {self.splits})")
        if not self.n:
            raise ValueError("no documents captured")
        self.flush()
        H, R, n = self.H, self.R, float(self.n)
        j = S - self.S0
        cx, s1x = self.cen[j], self.s1[j]
        G = self.acc[S]
        late = list(range(S, self.L))
        cy, sy, sxy = {}, {}, {}
        for i in late:
            c, s1y = self.cen[i - self.S0], self.s1[i - self.S0]
            blk = G[:, (i - S) * R:(i - S + 1) * R]
            cy[i] = c.c.to(device)
            sy[i] = (s1y - n * c.delta).to(device)
            sxy[i] = ridge.recentre(ridge.centred_products(blk, H, cx, H, c), s1x, s1y, cx.delta, c.delta, n).to(device)
        return dict(split=S, layers=late, dim=H, n=self.n, cx=cx.c.to(device), cy=cy,
                    sx=(s1x - n * cx.delta).to(device), sxx=sxy[S].clone(), sy=sy, sxy=sxy)


def fit_maps(state, lambdas=LAMBDAS, device="cuda"):
    """{lam: {layer: (W [d_out, d_in] bf16, b [d_out] bf16)}} on the device: RidgeFit of every late layer
    for every lambda, rounded to bf16 as the saved maps are (fit_sweep.py:286-293)."""
    fit = ridge.RidgeFit(state, device=device)
    per = fit.layers(state["layers"], lambdas)
    return {lam: {i: (per[i][lam][0].to(torch.bfloat16), per[i][lam][1].to(torch.bfloat16))
                  for i in state["layers"]} for lam in lambdas}


def _inputs(model, ids, first):
    got = {}
    model.forward_exact(ids, hook=lambda i, h: got.__setitem__(i, h) if i != "final" and i >= first else None,
                        stop=model.n_layers - 1)
    return got


def _read_groups(model, i):
    """(weights of layer i's reads, [(column, na, nb, d, gain, weight per row), ...]): an attention layer's
    reads are the pre-RoPE K | V of [W_k; W_v] (code/kva/model.py:282-287, :353-359, :558-565), one group pair
    with the k_norm gain on K; a GDN layer's are its in-projection outputs before the conv
    (code/kva/model.py:566-571): q | k per key head, v per value head, and the [b | a] row, from one product
    over [W_qkv; W_b; W_a]."""
    if model.layer_types[i] == "attn":
        w = model._layer(i)
        hkv, d = model.n_kv, model.head_dim
        return w["wkv"], [(0, hkv, hkv, d, w.get("k_norm"), 1.0 / hkv)]
    w = model._layer(i, "gdn")
    kd, vd, nv = model.nk * model.dk, model.nv * model.dv, model.nv
    if 2 * nv < 8 or 2 * nv > 256 or (2 * nv) & (2 * nv - 1):
        raise UnsupportedArchitecture(f"read scores of GDN layers with {nv} value heads (2 nv: a power of two, "
                                      f"8 to 256)")
    return w["w_in"], [(0, model.nk, model.nk, model.dk, None, 1.0 / model.nk), (2 * kd, nv, 0, model.dv, None, 1.0 / nv),
                       (2 * kd + vd, 1, 0, 2 * nv, None, 1.0)]


@torch.no_grad()
def read_scores(model, held, split, maps):
    """{candidate: {layer: mean read cosine}} over the held-out documents (fit_sweep.py:298-314);
    candidates: the lambdas of maps, then "identity". Per document and layer, the mean over the layer's
    reads (K and V; or q, k, v and [b | a]) of each read's mean cosine over rows and vectors."""
    late = list(range(split, model.n_layers))
    cand = list(maps) + ["identity"]
    dev = model.device
    score = torch.zeros(len(cand), len(late), 4, dtype=torch.float64, device=dev)
    nreads = []
    H = model.hidden
    for ids in held:
        got = _inputs(model, ids, split)
        hs = got[split]
        n = hs.shape[0]
        ws = torch.empty(8 * ((n + 15) // 16) + 8, dtype=torch.uint8, device=dev)
        ssq_s = ops.row_ssq(hs)
        nreads = []
        for j, i in enumerate(late):
            wr, groups = _read_groups(model, i)
            nreads.append(sum(1 + (nb > 0) for _, _, nb, _, _, _ in groups))
            gws = model.gemm_workspace(n, wr.shape[0], H, dev)
            true = ops.norm_linear(got[i], ops.row_ssq(got[i]), model.eps, wr, workspace=gws)
            pred = torch.empty_like(true)
            for c, lam in enumerate(cand):
                if lam == "identity":
                    x, sx = hs, ssq_s
                else:
                    W, b = maps[lam][i]
                    x, sx = ops.map_apply(hs, W, b, workspace=model.gemm_workspace(n, W.shape[0], H, dev))
                ops.norm_linear(x, sx, model.eps, wr, out=pred, workspace=gws)
                slot = 0
                for col, na, nb, d, gain, wt in groups:
                    width = (na + nb) * d
                    ops.read_cosine(pred[:, col:col + width], true[:, col:col + width], na, nb, d, gain,
                                    model.knorm_kind, wt / n, score[c, j, slot:slot + 2], workspace=ws)
                    slot += 1 + (nb > 0)
    div = torch.tensor(nreads, dtype=torch.float64, device=dev) * len(held)
    s = (score.sum(2) / div).cpu()
    return {lam: {i: float(s[c, j]) for j, i in enumerate(late)} for c, lam in enumerate(cand)}


def best_lambda(scores, lambdas=LAMBDAS):
    """The lambda with the highest mean score over layers, the first in lambdas order on ties
    (fit_sweep.py:315-318)."""
    mean = {c: sum(v.values()) / len(v) for c, v in scores.items()}
    return max(lambdas, key=lambda lam: mean[lam])


def fit_sweep(model, docs, held, splits, lambdas=LAMBDAS, block=BLOCK):
    """Capture over docs, then per split: fit every lambda, pick one by the held-out read cosine, and
    return {S: dict(projector=Projector(S, W, b) of the chosen lambda (bf16, on the device), lam, scores,
    rows)} (fit_sweep.py:236-337 without the files)."""
    cap = Capture(model, splits, block)
    for ids in docs:
        cap.add_document(ids)
    out = {}
    for S in sorted(cap.splits, reverse=True):
        maps = fit_maps(cap.state(S, device=model.device), lambdas, device=model.device)
        scores = read_scores(model, held, S, maps)
        lam = best_lambda(scores, lambdas)
        W = {i: w for i, (w, _) in maps[lam].items()}
        B = {i: b for i, (_, b) in maps[lam].items()}
        out[S] = dict(projector=Projector(S, W, B, dict(lam=lam, rows=cap.n, taps=S, sweep=True, docs=cap.docs)),
                      lam=lam, scores=scores, rows=cap.n)
    return out
