"""Oracle numerical primitives (test infrastructure; see oracle/__init__.py).

Restates code/kva/ops.py of the reference with the same dtype semantics: every op that the reference
runs in the activation dtype rounds to that dtype at the same point, fp32 work stays fp32.
Layouts: activations [tokens, features]; per-head tensors [heads, tokens, dim]; GDN state
[value_heads, key_dim, value_dim] fp32; conv state [kernel - 1, channels].
"""
import math

import torch
import torch.nn.functional as F


def _inv_rms(xf, eps):
    """1 / sqrt(mean(x^2) + eps) over the last dim, fp32."""
    return torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)


def rms_norm(x, weight, eps):
    """Llama RMSNorm (code/kva/ops.py:14-18): normalise in fp32, round to x.dtype, then multiply by
    the weight in x.dtype (two roundings for bf16)."""
    normed = (x.float() * _inv_rms(x.float(), eps)).to(x.dtype)
    return weight * normed


def rms_norm_zc(x, weight, eps):
    """Qwen3.5 zero-centred RMSNorm (code/kva/ops.py:21-25): scale by (1 + w) in fp32, one rounding."""
    xf = x.float()
    return (xf * _inv_rms(xf, eps) * (1.0 + weight.float())).to(x.dtype)


def rms_norm_gated(x, gate, weight, eps):
    """GDN output norm (code/kva/ops.py:28-33): RMSNorm, weight in x.dtype, times silu(gate) in fp32."""
    y = weight * (x.float() * _inv_rms(x.float(), eps)).to(x.dtype)
    return (y * F.silu(gate.float())).to(x.dtype)


def l2norm(x, eps=1e-6):
    """x / sqrt(sum(x^2) + eps) over the last dim (code/kva/ops.py:36-37)."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


# ---------------------------------------------------------------------------------------------- RoPE

def inv_freq_default(theta, rot_dim):
    """theta^(-2j/rot) for j < rot/2, fp32 (code/kva/ops.py:42-43)."""
    expo = torch.arange(0, rot_dim, 2, dtype=torch.float32) / rot_dim
    return 1.0 / (theta ** expo)


def inv_freq_llama3(theta, dim, factor, low_freq_factor, high_freq_factor, original_max):
    """Llama-3.1 frequency rescale (code/kva/ops.py:46-56): long wavelengths divided by `factor`,
    short ones kept, the band between blended linearly in original_max / wavelength."""
    base = inv_freq_default(theta, dim)
    wavelen = 2 * math.pi / base
    long_wl = original_max / low_freq_factor
    short_wl = original_max / high_freq_factor
    out = torch.where(wavelen > long_wl, base / factor, base)
    t = (original_max / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    blended = (1 - t) * out / factor + t * out
    band = (wavelen >= short_wl) & (wavelen <= long_wl)
    return torch.where(band, blended, out)


def rope_cos_sin(inv_freq, positions, dtype):
    """cos / sin [tokens, rot] (code/kva/ops.py:59-63): angle = float(pos) * inv_freq in fp32, the
    half-table repeated twice, cos and sin in fp32, then rounded to `dtype`."""
    ang = positions.float()[:, None] * inv_freq.to(positions.device)[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def rotate_half(x):
    """Half-split rotation [x1, x2] -> [-x2, x1] (code/kva/ops.py:66-68), not interleaved pairs."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x, cos, sin):
    """x [heads, tokens, d] rotated on its first cos.shape[-1] dims, the rest passed through
    (code/kva/ops.py:71-77); each product and the sum round to x.dtype."""
    rot = cos.shape[-1]
    head, tail = x[..., :rot], x[..., rot:]
    turned = head * cos + rotate_half(head) * sin
    return turned if rot == x.shape[-1] else torch.cat((turned, tail), dim=-1)


# ------------------------------------------------------------------------------------------ attention

def attend_at(q, k, v, scale, qpos):
    """Causal GQA attention of queries at positions qpos over keys 0..nk-1 (query t sees key j when
    j <= qpos[t]); scores and softmax fp32, probabilities rounded to v.dtype before P.V
    (code/kva/ops.py:90-152, unblocked: the reference's query blocking is a memory bound only).
    q [Hq, nq, d], k / v [Hkv, nk, d] -> [nq, Hq * dv]."""
    hq, nq, d = q.shape
    hkv, nk, _ = k.shape
    rep = hq // hkv
    s = torch.matmul(q.reshape(hkv, rep * nq, d).float(), k.float().transpose(1, 2)) * scale
    s = s.view(hkv, rep, nq, nk)
    future = torch.arange(nk)[None, :] > qpos.to(torch.long)[:, None]
    s = s.masked_fill(future, float("-inf"))
    p = torch.softmax(s, -1).to(v.dtype).view(hkv, rep * nq, nk)
    o = torch.matmul(p, v).view(hq, nq, -1)
    return o.transpose(0, 1).reshape(nq, -1)


def attend(q, k, v, scale):
    """Queries that are the last q.shape[1] positions of the keys (bottom-right causal)."""
    nk, nq = k.shape[1], q.shape[1]
    return attend_at(q, k, v, scale, torch.arange(nk - nq, nk))


# -------------------------------------------------------------------------------------- GDN primitives

def causal_conv(x, state, weight):
    """Depthwise causal conv + SiLU (code/kva/ops.py:173-186). x [n, C] pre-conv rows, state
    [K-1, C] (None: zeros), weight [C, K]. Accumulates tap by tap in fp32 (tap j reads row t + j of
    [state; x]), SiLU, rounds to x.dtype. New state = the last K-1 rows of [state; x]."""
    taps = weight.shape[1]
    n, c = x.shape
    prev = torch.zeros(taps - 1, c, dtype=x.dtype) if state is None else state.to(x.dtype)
    seq = torch.cat((prev, x), 0)
    wf = weight.float()
    acc = torch.zeros(n, c, dtype=torch.float32)
    for j in range(taps):
        acc = acc + seq[j:j + n].float() * wf[:, j]
    return F.silu(acc).to(x.dtype), seq[seq.shape[0] - (taps - 1):].clone()


def unit_lower_inverse(a):
    """(I + A)^-1 for strictly lower-triangular A [..., C, C] by forward substitution row by row
    (code/kva/ops.py:189-196): row i of T = -A_i - sum_{j<i} A_ij T_j restricted to columns < i."""
    c = a.shape[-1]
    t = -a.clone()
    for i in range(1, c):
        r = t[..., i, :i].clone()
        t[..., i, :i] = r + torch.einsum("...j,...jk->...k", r, t[..., :i, :i])
    return t + torch.eye(c, dtype=a.dtype)


def delta_rule(q, k, v, g, beta, state=None, chunk=64, segment=4096, checkpoint_every=None, offset=0,
               need_out=True):
    """Chunked gated delta rule in fp32 (code/kva/ops.py:199-262).

    Recurrence per token t (S [H, dk, dv]): S <- e^{g_t} S; S <- S + k_t (beta_t (v_t - S^T k_t))^T;
    o_t = S^T q_t. Chunk form: within a chunk, gamma = cumsum(g); A = tril_{-1}(beta K K^T e^{gamma_i -
    gamma_j}); T = (I + A)^-1; U = T (beta V); W = T (beta e^gamma K); per chunk v_new = U - W S,
    S <- e^{gamma_last} S + (K e^{gamma_last - gamma})^T v_new. The chunk grid starts at this call's
    first token and restarts at every `segment` boundary; a short chunk is zero-padded (g = 0, beta = 0
    padding leaves the state unchanged). Returns (out [H, n, dv] fp32 or None, state, checkpoints)."""
    h, n, dk = k.shape
    dv = v.shape[-1]
    s = torch.zeros(h, dk, dv) if state is None else state.float().clone()
    out = torch.empty(h, n, dv) if need_out else None
    ckpts = {}
    if checkpoint_every:
        assert checkpoint_every % chunk == 0 and segment % chunk == 0
    lower_incl = torch.ones(chunk, chunk, dtype=torch.bool).tril()
    for a0 in range(0, n, segment):
        a1 = min(n, a0 + segment)
        m = a1 - a0
        nc = -(-m // chunk)
        pad = nc * chunk - m

        def cut(t):
            t = t[:, a0:a1].float()
            if pad:
                t = torch.cat((t, t.new_zeros((h, pad) + tuple(t.shape[2:]))), 1)
            return t.reshape((h, nc, chunk) + tuple(t.shape[2:]))

        qc, kc, vc, gc, bc = cut(q), cut(k), cut(v), cut(g), cut(beta)
        gam = gc.cumsum(-1)
        gap = gam[..., :, None] - gam[..., None, :]
        decay = torch.where(lower_incl, gap, torch.full_like(gap, float("-inf"))).exp()
        a = (bc[..., :, None] * (kc @ kc.transpose(-1, -2)) * decay).tril(-1)
        t = unit_lower_inverse(a)
        u = t @ (bc[..., None] * vc)
        w = t @ (bc[..., None] * gam.exp()[..., None] * kc)
        k_to_end = kc * (gam[..., -1:] - gam).exp()[..., None]
        tot = gam[..., -1].exp()
        if need_out:
            qk = (qc @ kc.transpose(-1, -2)) * decay
            q_dec = qc * gam.exp()[..., None]
        for c in range(nc):
            v_new = u[:, c] - w[:, c] @ s
            if need_out:
                o = q_dec[:, c] @ s + qk[:, c] @ v_new
                lo = a0 + c * chunk
                hi = min(a1, lo + chunk)
                out[:, lo:hi] = o[:, :hi - lo]
            s = s * tot[:, c, None, None] + k_to_end[:, c].transpose(-1, -2) @ v_new
            done = a0 + (c + 1) * chunk
            if checkpoint_every and done <= n and done % checkpoint_every == 0:
                ckpts[offset + done] = s.clone()
    return out, s, ckpts


def delta_rule_recurrent(q, k, v, g, beta, state=None):
    """Token-by-token gated delta rule (code/kva/ops.py:265-277): the closed form the chunked rule
    must equal. Returns (out [H, n, dv] fp32, final state)."""
    h, n, dk = k.shape
    dv = v.shape[-1]
    s = torch.zeros(h, dk, dv) if state is None else state.float().clone()
    out = torch.empty(h, n, dv)
    for t in range(n):
        s = s * g[:, t].float().exp()[:, None, None]
        kt, vt, qt = k[:, t].float(), v[:, t].float(), q[:, t].float()
        err = vt - torch.einsum("hkv,hk->hv", s, kt)
        s = s + kt[:, :, None] * (beta[:, t].float()[:, None] * err)[:, None, :]
        out[:, t] = torch.einsum("hkv,hk->hv", s, qt)
    return out, s
