"""Pins the oracle's GDN primitives and RoPE tables by closed forms and library routines."""
import math

import torch

from oracle import ops


def _gdn_inputs(h=3, n=200, dk=16, dv=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = ops.l2norm(torch.randn(h, n, dk, generator=g)) * dk ** -0.5
    k = ops.l2norm(torch.randn(h, n, dk, generator=g))
    v = torch.randn(h, n, dv, generator=g)
    gate = -torch.rand(h, n, generator=g) * 0.5
    beta = torch.rand(h, n, generator=g)
    s0 = torch.randn(h, dk, dv, generator=g) * 0.1
    return q, k, v, gate, beta, s0


def test_delta_rule_matches_recurrence():
    """Chunked form == token-by-token recurrence (code/tests/test_ops.py:19-24)."""
    q, k, v, g, b, s0 = _gdn_inputs()
    ref, sref = ops.delta_rule_recurrent(q, k, v, g, b, s0)
    out, s, _ = ops.delta_rule(q, k, v, g, b, s0, chunk=16, segment=64)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(s, sref, atol=1e-5, rtol=1e-5)


def test_delta_rule_checkpoints_and_continuation():
    """Checkpoints equal the recurrence at those tokens; a second call continuing from the first's
    state equals one call (code/tests/test_ops.py:27-38)."""
    q, k, v, g, b, s0 = _gdn_inputs(n=192)
    _, _, ck = ops.delta_rule(q, k, v, g, b, s0, chunk=16, segment=64, checkpoint_every=32, need_out=False)
    for t in (32, 96, 192):
        _, s_t = ops.delta_rule_recurrent(q[:, :t], k[:, :t], v[:, :t], g[:, :t], b[:, :t], s0)
        torch.testing.assert_close(ck[t], s_t, atol=1e-5, rtol=1e-5)
    o1, s1, _ = ops.delta_rule(q[:, :77], k[:, :77], v[:, :77], g[:, :77], b[:, :77], s0, chunk=16)
    o2, s2, _ = ops.delta_rule(q[:, 77:], k[:, 77:], v[:, 77:], g[:, 77:], b[:, 77:], s1, chunk=16)
    ref, sref = ops.delta_rule_recurrent(q, k, v, g, b, s0)
    torch.testing.assert_close(torch.cat((o1, o2), 1), ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(s2, sref, atol=1e-5, rtol=1e-5)


def test_delta_rule_special_cases():
    """beta = 0 and g = 0: the state never changes. One token from a zero state with beta = 1:
    S = k v^T (a rank-1 write), o = (q.k) v."""
    q, k, v, g, b, s0 = _gdn_inputs(n=40)
    _, s, _ = ops.delta_rule(q, k, v, torch.zeros_like(g), torch.zeros_like(b), s0, chunk=16)
    torch.testing.assert_close(s, s0)
    out, s = ops.delta_rule_recurrent(q[:, :1], k[:, :1], v[:, :1], torch.zeros(3, 1), torch.ones(3, 1))
    torch.testing.assert_close(s, k[:, 0, :, None] * v[:, 0, None, :])
    torch.testing.assert_close(out[:, 0], (q[:, 0] * k[:, 0]).sum(-1, keepdim=True) * v[:, 0])


def test_unit_lower_inverse_is_the_inverse():
    a = torch.randn(4, 24, 24, generator=torch.Generator().manual_seed(1)).tril(-1) * 0.3
    t = ops.unit_lower_inverse(a)
    torch.testing.assert_close(t @ (torch.eye(24) + a), torch.eye(24).expand(4, 24, 24), atol=1e-5, rtol=0)


def test_causal_conv_is_conv1d_and_continues():
    """One call == two chained calls == F.conv1d(padding=K-1, groups=C) + SiLU (code/tests/test_ops.py:41-51)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(50, 12, generator=g)
    w = torch.randn(12, 4, generator=g)
    full, st = ops.causal_conv(x, None, w)
    a, sa = ops.causal_conv(x[:20], None, w)
    b, sb = ops.causal_conv(x[20:], sa, w)
    torch.testing.assert_close(torch.cat((a, b)), full)
    torch.testing.assert_close(sb, st)
    torch.testing.assert_close(st, x[-3:])
    ref = torch.nn.functional.conv1d(x.T[None], w[:, None], padding=3, groups=12)[0, :, :50].T
    torch.testing.assert_close(full, torch.nn.functional.silu(ref), atol=1e-6, rtol=1e-5)


def test_inv_freq_and_rope_tables():
    """inv_freq_default is theta^(-2j/d); the llama3 rescale leaves short wavelengths alone and divides
    long ones by the factor; cos/sin tables are the textbook angles with the half table repeated."""
    f = ops.inv_freq_default(10000.0, 64)
    torch.testing.assert_close(f, torch.tensor([10000.0 ** (-2 * j / 64) for j in range(32)]), atol=0, rtol=1e-6)
    l3 = ops.inv_freq_llama3(500000.0, 128, 8.0, 1.0, 4.0, 8192)
    base = ops.inv_freq_default(500000.0, 128)
    wl = 2 * math.pi / base
    assert torch.equal(l3[wl < 8192 / 4], base[wl < 8192 / 4])
    torch.testing.assert_close(l3[wl > 8192], base[wl > 8192] / 8)
    cos, sin = ops.rope_cos_sin(f, torch.arange(5), torch.float32)
    ang = torch.arange(5).float()[:, None] * f[None]
    torch.testing.assert_close(cos, torch.cat((ang.cos(), ang.cos()), -1))
    torch.testing.assert_close(sin, torch.cat((ang.sin(), ang.sin()), -1))


def test_apply_rope_is_a_rotation_per_pair():
    """Rotating pairs (j, j + d/2) by the angle: norms kept, pos 0 is the identity, partial RoPE leaves
    the trailing dims."""
    x = torch.randn(2, 6, 32, generator=torch.Generator().manual_seed(3))
    f = ops.inv_freq_default(1e4, 16)
    cos, sin = ops.rope_cos_sin(f, torch.arange(6), torch.float32)
    y = ops.apply_rope(x, cos, sin)
    torch.testing.assert_close(y[..., :16].norm(dim=-1), x[..., :16].norm(dim=-1))
    torch.testing.assert_close(y[:, 0], x[:, 0])
    assert torch.equal(y[..., 16:], x[..., 16:])
    a = torch.arange(6).float()[:, None] * f[None]
    z = torch.complex(x[..., :8], x[..., 8:16]) * torch.polar(torch.ones_like(a), a)
    torch.testing.assert_close(y[..., :8], z.real, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(y[..., 8:16], z.imag, atol=1e-5, rtol=1e-5)
