"""Pins the oracle's model math against transformers' own implementations (fp32, CPU): logits of the
whole forward, and -- the fill path itself -- each layer's cache written from the true layer inputs:
post-RoPE K and V of attention layers, conv and recurrent state of GDN layers. Positive controls show
each comparison resolves the convention it pins (rotation layout, llama3 rescale, k_norm, gate formula)."""
import pytest
import torch

from conftest import ids_of
from oracle import model as OM
from oracle import ops

TOL = dict(atol=2e-4, rtol=2e-4)


def rel_err(a, b):
    """Relative Frobenius error |a - b| / |b|."""
    return float((a.double() - b.double()).norm() / b.double().norm())


def _hf_run(hf, ids):
    with torch.no_grad():
        out = hf(ids[None], use_cache=True, output_hidden_states=True)
    return out.logits[0].float(), out.hidden_states, out.past_key_values


@pytest.mark.parametrize("name", ["hf_llama", "hf_qwen3", "hf_qwen35"])
def test_forward_matches_transformers(name, request):
    hf = request.getfixturevalue(name)
    m = OM.OracleModel.from_hf(hf)
    ids = ids_of(150)
    mine, _ = m.forward_exact(ids, keep=torch.arange(150))
    ref, _, _ = _hf_run(hf, ids)
    torch.testing.assert_close(mine, ref, **TOL)


def _fill_matches_cache(m, hidden, cache_hf, n):
    pos = torch.arange(n)
    for i in range(m.n_layers):
        c = m.new_cache()
        m.fill(i, hidden[i][0], pos, c)
        layer = cache_hf.layers[i]
        if m.layer_types[i] == "attn":
            torch.testing.assert_close(c[i]["k"], layer.keys[0], atol=1e-5, rtol=1e-5)
            torch.testing.assert_close(c[i]["v"], layer.values[0], atol=1e-5, rtol=1e-5)
            assert c[i]["n"] == n and c[i]["kbuf"].shape[1] == n + OM.KV_RESERVE
        else:
            conv = layer.conv_states[0][0]                         # [C, K]: the last K pre-conv rows
            torch.testing.assert_close(c[i]["conv"], conv[:, 1:].T, atol=1e-6, rtol=1e-6)
            ref = layer.recurrent_states[0][0]
            assert rel_err(c[i]["rec"], ref) < 1e-5, (i, rel_err(c[i]["rec"], ref))
            assert c[i]["len"] == n


@pytest.mark.parametrize("name", ["hf_llama", "hf_qwen3", "hf_qwen35"])
def test_fill_writes_transformers_cache(name, request):
    """fill(i, true layer-i input) == the cache transformers' exact layer wrote (code/tests/test_qwen3.py:117-128
    states this for the reference's own layer; here it pins the oracle against an independent implementation)."""
    hf = request.getfixturevalue(name)
    m = OM.OracleModel.from_hf(hf)
    n = 130
    _, hidden, cache = _hf_run(hf, ids_of(n, 7))
    _fill_matches_cache(m, hidden, cache, n)


def test_positive_control_rotation_layout(hf_llama, monkeypatch):
    """Interleaved-pair rotation instead of the half split must NOT match: the K comparison resolves it."""
    m = OM.OracleModel.from_hf(hf_llama)
    _, hidden, cache = _hf_run(hf_llama, ids_of(80, 1))

    def interleaved(x):
        return torch.stack((-x[..., 1::2], x[..., ::2]), -1).flatten(-2)
    monkeypatch.setattr(ops, "rotate_half", interleaved)
    c = m.new_cache()
    m.fill(0, hidden[0][0], torch.arange(80), c)
    assert (c[0]["k"] - cache.layers[0].keys[0]).abs().max() > 1e-3


def test_positive_control_llama3_rescale(hf_llama):
    """Default inverse frequencies instead of the llama3 rescale must NOT match (positions exceed the
    fixture's original_max 64)."""
    m = OM.OracleModel.from_hf(hf_llama)
    _, hidden, cache = _hf_run(hf_llama, ids_of(120, 2))
    m.inv_freq = ops.inv_freq_default(500000.0, m.head_dim)
    c = m.new_cache()
    m.fill(0, hidden[0][0], torch.arange(120), c)
    assert (c[0]["k"] - cache.layers[0].keys[0]).abs().max() > 1e-4


def test_positive_control_k_norm(hf_qwen3):
    """Qwen3 without the per-head k_norm (Llama's K) must NOT match."""
    m = OM.OracleModel.from_hf(hf_qwen3)
    _, hidden, cache = _hf_run(hf_qwen3, ids_of(60, 3))
    m.arch = "llama"
    c = m.new_cache()
    m.fill(0, hidden[0][0], torch.arange(60), c)
    assert (c[0]["k"] - cache.layers[0].keys[0]).abs().max() > 1e-3


def test_positive_control_gdn_decay(hf_qwen35):
    """A decay without the softplus (g = -exp(A_log) (a + dt_bias)) must NOT match the recurrent state."""
    m = OM.OracleModel.from_hf(hf_qwen35)
    _, hidden, cache = _hf_run(hf_qwen35, ids_of(90, 4))
    c = m.new_cache()
    orig = OM.F.softplus
    try:
        OM.F.softplus = lambda t: t
        m.fill(0, hidden[0][0], torch.arange(90), c)
    finally:
        OM.F.softplus = orig
    assert rel_err(c[0]["rec"], cache.layers[0].recurrent_states[0][0]) > 1e-2


def test_gdn_row_segments_match(hf_qwen35):
    """Segmenting the GDN rows (GDN_ROWS) leaves results unchanged (code/tests/test_model.py:46-59)."""
    m = OM.OracleModel.from_hf(hf_qwen35)
    ids = ids_of(300, 5)
    ref, c1 = m.forward_exact(ids, keep=torch.arange(300), gdn_checkpoint_every=64)
    old = OM.GDN_ROWS
    try:
        OM.GDN_ROWS = 128
        seg, c2 = m.forward_exact(ids, keep=torch.arange(300), gdn_checkpoint_every=64)
    finally:
        OM.GDN_ROWS = old
    torch.testing.assert_close(seg, ref, atol=1e-5, rtol=1e-5)
    assert sorted(c1[0]["checkpoints"]) == sorted(c2[0]["checkpoints"]) == [64, 128, 192, 256]


@pytest.mark.parametrize("name", ["hf_qwen3", "hf_qwen35"])
def test_cached_decode_matches_full(name, request):
    """Prefill then token-by-token decode equals one full forward (code/tests/test_model.py:29-43)."""
    m = OM.OracleModel.from_hf(request.getfixturevalue(name))
    ids = ids_of(140, 3)
    full, _ = m.forward_exact(ids, keep=torch.arange(140))
    _, cache = m.forward_exact(ids[:130])
    rows = []
    for t in range(130, 140):
        h = m.embed(ids[t:t + 1])
        for i in range(m.n_layers):
            h = m.layer(i, h, torch.tensor([t]), cache)
        rows.append(m.logits(h))
    torch.testing.assert_close(torch.cat(rows), full[130:], atol=1e-4, rtol=1e-4)


def test_fill_kv_equals_fill(hf_llama):
    """fill_kv from the pre-RoPE K / V of the normed inputs writes what fill writes (code/kva/model.py:161-165)."""
    m = OM.OracleModel.from_hf(hf_llama)
    x = torch.randn(40, m.hidden, generator=torch.Generator().manual_seed(9))
    pos = torch.arange(40)
    a, b = m.new_cache(), m.new_cache()
    m.fill(2, x, pos, a)
    xn = m.in_norm(x, m.W[2]["ln1"])
    k = torch.nn.functional.linear(xn, m.W[2]["k"]).view(40, m.n_kv, m.head_dim)
    v = torch.nn.functional.linear(xn, m.W[2]["v"]).view(40, m.n_kv, m.head_dim)
    m.fill_kv(2, k, v, pos, b)
    assert torch.equal(a[2]["k"], b[2]["k"]) and torch.equal(a[2]["v"], b[2]["v"])


def test_append_kv_grows_with_reserve():
    c = {}
    k = torch.randn(2, 10, 4)
    OM.OracleModel.append_kv(c, k, k + 1)
    assert c["kbuf"].shape[1] == 10 + OM.KV_RESERVE and c["n"] == 10
    OM.OracleModel.append_kv(c, k[:, :5], k[:, :5])
    assert c["kbuf"].shape[1] == 10 + OM.KV_RESERVE and c["n"] == 15
    big = torch.randn(2, 100, 4)
    OM.OracleModel.append_kv(c, big, big)
    assert c["kbuf"].shape[1] == 115 + OM.KV_RESERVE and torch.equal(c["k"][:, :10], k)
    assert torch.equal(c["k"][:, 15:], big)
