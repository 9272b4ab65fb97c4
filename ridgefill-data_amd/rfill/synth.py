"""Seeded synthetic workloads for the fill (no checkpoints or datasets are used).

  dense_fill(...)  Llama-3.1-8B / Qwen3-8B shaped late-layer fill: split-layer hidden states h_split
                   [N, H] bf16 = N(0, 1) rows x a per-channel log-normal(0, 0.5) gain, 4 outlier
                   channels x 20; per late layer l a ridge map W_l = I + 0.02 N(0, 1/H) (variance 1/H)
                   with bias N(0, 1e-3) (std), an input RMSNorm gain 1 + N(0, 0.05), K / V projections
                   N(0, 0.02) and, for Qwen3, a k_norm gain 1 + N(0, 0.05).
  hybrid_fill(...) the Gated-DeltaNet hybrid (Qwen3.5-shaped, hidden 2048, layers 3 GDN : 1 attention)
                   late-layer fill: the same h_split and ridge maps at H = 2048; zero-centred input-norm
                   gains N(0, 0.05); GDN in-projections (q | k | v [8192, 2048], b, a [32, 2048])
                   N(0, 0.02), depthwise conv U(-0.5, 0.5) [8192, 4], A_log = log U(0, 16) and
                   dt_bias = 1 (the architecture's own initialisation), so the gates run through the
                   checkpoint formula g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b);
                   attention layers K / V N(0, 0.02) with a zero-centred k_norm gain N(0, 0.05). With
                   full=True also the rest of each late layer for the exact tail (hybrid_full_weights; MLP
                   width 6144, which the hybrid's description leaves open).
  full_model(...)  every layer's whole weights, the head and an N(0, 1) embedding table (the exact forward
                   of the capture and the lambda selection).
Seeds: 10 (rows), 11 (channel gains and outliers), 12 + l (layer l's weights), 100 + l (the map of
hybrid GDN layer l), 13 (exact-row positions), 14 (exact-row inputs), 16 (embedding table). Normal(mu, s) parameters are standard deviations except the
explicit variance 1/H of the map noise.
"""
import torch

LLAMA_8B = dict(model_type="llama", num_hidden_layers=32, hidden_size=4096, num_attention_heads=32,
                num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, intermediate_size=14336,
                vocab_size=128256)
QWEN3_8B = dict(model_type="qwen3", num_hidden_layers=36, hidden_size=4096, num_attention_heads=32,
                num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, intermediate_size=12288, vocab_size=151936,
                rope_parameters=dict(rope_type="default", rope_theta=1000000.0))


QWEN35_HYBRID = dict(model_type="qwen3_5_text", num_hidden_layers=48, hidden_size=2048, num_attention_heads=16,
                     num_key_value_heads=2, head_dim=256, rms_norm_eps=1e-6,
                     layer_types=["full_attention" if i % 4 == 3 else "linear_attention" for i in range(48)],
                     linear_num_key_heads=16, linear_num_value_heads=32, linear_key_head_dim=128,
                     linear_value_head_dim=128, linear_conv_kernel_dim=4,
                     rope_parameters=dict(rope_type="default", rope_theta=10000000.0, partial_rotary_factor=0.25),
                     intermediate_size=6144)


def _gen(seed, device):
    return torch.Generator(device=device).manual_seed(seed)


def hidden_states(n, h, device="cpu", seed_rows=10, seed_gain=11, outliers=4, outlier_scale=20.0):
    """[n, h] bf16 split-layer rows: N(0, 1) x log-normal(0, 0.5) channel gain, `outliers` channels x 20."""
    g = _gen(seed_gain, "cpu")
    gain = torch.exp(0.5 * torch.randn(h, generator=g))
    pick = torch.randperm(h, generator=g)[:outliers]
    gain[pick] *= outlier_scale
    rows = torch.randn(n, h, generator=_gen(seed_rows, device), device=device)
    return (rows * gain.to(device)).to(torch.bfloat16)


def layer_weights(cfg, layer, device="cpu", map_noise=0.02, with_map=True, full=False):
    """HF-named weights of one late attention layer plus its ridge map (W, c), seed 12 + layer. full: also
    the rest of the layer the exact rows run through (q / o projections, q_norm, the post-attention norm,
    the SwiGLU MLP; matrices N(0, 0.02), norm gains 1 + N(0, 0.05)), drawn after the fill's weights."""
    h, hkv, d = cfg["hidden_size"], cfg["num_key_value_heads"], cfg["head_dim"]
    g = _gen(12 + layer, device)
    p = f"model.layers.{layer}."
    rn = lambda *s: torch.randn(*s, generator=g, device=device)                        # noqa: E731
    t = {
        p + "input_layernorm.weight": 1 + 0.05 * rn(h),
        p + "self_attn.k_proj.weight": 0.02 * rn(hkv * d, h),
        p + "self_attn.v_proj.weight": 0.02 * rn(hkv * d, h),
    }
    if cfg["model_type"] != "llama":
        t[p + "self_attn.k_norm.weight"] = 1 + 0.05 * rn(d)
    w = c = None
    if with_map:
        w = (torch.eye(h, device=device) + map_noise * rn(h, h) / h ** 0.5).to(torch.bfloat16)
        c = (1e-3 * rn(h)).to(torch.bfloat16)
    if full:
        hq, inter = cfg["num_attention_heads"], cfg["intermediate_size"]
        t[p + "self_attn.q_proj.weight"] = 0.02 * rn(hq * d, h)
        t[p + "self_attn.o_proj.weight"] = 0.02 * rn(h, hq * d)
        if cfg["model_type"] != "llama":
            t[p + "self_attn.q_norm.weight"] = 1 + 0.05 * rn(d)
        t[p + "post_attention_layernorm.weight"] = 1 + 0.05 * rn(h)
        t[p + "mlp.gate_proj.weight"] = 0.02 * rn(inter, h)
        t[p + "mlp.up_proj.weight"] = 0.02 * rn(inter, h)
        t[p + "mlp.down_proj.weight"] = 0.02 * rn(h, inter)
    t = {k: v.to(torch.bfloat16) for k, v in t.items()}
    return t, w, c


def head_weights(cfg, device="cpu"):
    """The final norm gain 1 + N(0, 0.05) and lm_head N(0, 0.02) [vocab, H] (seed 15), bf16."""
    h, vocab = cfg["hidden_size"], cfg["vocab_size"]
    g = _gen(15, device)
    return {"model.norm.weight": (1 + 0.05 * torch.randn(h, generator=g, device=device)).to(torch.bfloat16),
            "lm_head.weight": (0.02 * torch.randn(vocab, h, generator=g, device=device)).to(torch.bfloat16)}


def full_model(cfg, device="cpu"):
    """HF-named weights of every layer (layer_weights(full=True), seed 12 + l), the head (seed 15) and
    an embedding table N(0, 1) [vocab, H] (seed 16), bf16: the whole model an exact forward runs."""
    t = {}
    for l in range(cfg["num_hidden_layers"]):
        t.update(layer_weights(cfg, l, device, with_map=False, full=True)[0])
    t.update(head_weights(cfg, device))
    g = _gen(16, device)
    t["model.embed_tokens.weight"] = torch.randn(cfg["vocab_size"], cfg["hidden_size"], generator=g,
                                                 device=device).to(torch.bfloat16)
    return t


def dense_fill(cfg, split, n_rows, tail, device="cpu", exact_frac=0.0, with_maps=True, full=False, head=False):
    """A late-layer fill workload: dict(cfg, split, layers, h_split [n, H], P, tensors (HF names),
    maps {l: W}, biases {l: c}, rows (sorted exact-row positions < P), hr [|rows|, H]). full: the late
    layers' whole weights (for exact rows and the exact tail run through their layers); head: the final
    norm and lm_head (for the tail's logits)."""
    L, h = cfg["num_hidden_layers"], cfg["hidden_size"]
    layers = list(range(split, L))
    tensors, maps, biases = {}, {}, {}
    for l in layers:
        t, w, c = layer_weights(cfg, l, device, with_map=with_maps, full=full)
        tensors.update(t)
        if with_maps:
            maps[l], biases[l] = w, c
    if head:
        tensors.update(head_weights(cfg, device))
    P = n_rows - tail
    n_exact = int(round(exact_frac * P))
    rows = torch.randperm(P, generator=_gen(13, "cpu"))[:n_exact].sort().values
    hr = hidden_states(n_exact, h, device=device, seed_rows=14) if n_exact else None
    return dict(cfg=cfg, split=split, layers=layers, h_split=hidden_states(n_rows, h, device=device), P=P,
                tensors=tensors, maps=maps, biases=biases, rows=rows.to(device), hr=hr)


def student_t(shape, nu, generator, device):
    """Student-t(nu) samples z / sqrt(chi2_nu / nu), chi2 from nu squared normals (nu integer)."""
    z = torch.randn(shape, generator=generator, device=device)
    chi2 = torch.zeros(shape, device=device)
    for _ in range(nu):
        chi2 += torch.randn(shape, generator=generator, device=device) ** 2
    return z * torch.rsqrt(chi2 / nu)


def fit_maps(d, targets, device="cpu", scale=0.05):
    """The fit workload's true maps T_l = I + scale N(0, 1/d) (variance 1/d), seed 21 + l."""
    return [torch.eye(d, device=device) + scale * torch.randn(d, d, generator=_gen(21 + l, device), device=device)
            / d ** 0.5 for l in range(targets)]


def fit_chunk(chunk, rows, d, maps, device="cpu", nu=5, outliers=4, noise=0.1):
    """Rows [chunk * rows, (chunk + 1) * rows) of the fit workload: X = Student-t(nu) per element (seed
    20 + 1000 chunk) with `outliers` channels x 20 (seed 20), Y_l = X T_l + N(0, noise) (seed
    21 + l + 1000 chunk); bf16 storage, Y computed from the bf16 X in fp32."""
    g = _gen(20, "cpu")
    pick = torch.randperm(d, generator=g)[:outliers].to(device)
    x = student_t((rows, d), nu, _gen(20 + 1000 * chunk, device), device)
    x[:, pick] *= 20.0
    x = x.to(torch.bfloat16)
    ys = []
    for l, t in enumerate(maps):
        e = noise * torch.randn(rows, d, generator=_gen(21 + l + 1000 * chunk, device), device=device)
        ys.append((x.float() @ t + e).to(torch.bfloat16))
    return x, ys


def gdn_layer_weights(cfg, layer, device="cpu"):
    """HF-named weights of one Gated DeltaNet layer (seed 12 + layer)."""
    h, nk, nv = cfg["hidden_size"], cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    dk, dv, kc = cfg["linear_key_head_dim"], cfg["linear_value_head_dim"], cfg["linear_conv_kernel_dim"]
    C = 2 * nk * dk + nv * dv
    g = _gen(12 + layer, device)
    p = f"model.layers.{layer}."
    a = p + "linear_attn."
    rn = lambda *s: torch.randn(*s, generator=g, device=device)                        # noqa: E731
    t = {p + "input_layernorm.weight": 0.05 * rn(h), a + "in_proj_qkv.weight": 0.02 * rn(C, h),
         a + "in_proj_b.weight": 0.02 * rn(nv, h), a + "in_proj_a.weight": 0.02 * rn(nv, h),
         a + "conv1d.weight": torch.rand(C, 1, kc, generator=g, device=device) - 0.5}
    t = {k: v.to(torch.bfloat16) for k, v in t.items()}
    t[a + "A_log"] = torch.log(16 * torch.rand(nv, generator=g, device=device).clamp_min(1e-6))
    t[a + "dt_bias"] = torch.ones(nv, device=device)
    return t


def hybrid_full_weights(cfg, layer, device="cpu"):
    """The rest of a hybrid layer the exact tail runs through (seed 200 + layer): the SwiGLU MLP and its
    zero-centred post norm; attention: the gated q projection [2 hq d, H], o_proj, q_norm; GDN: the z
    projection, the gated output norm's weight 1 + N(0, 0.05), out_proj. Matrices N(0, 0.02), zero-centred
    norm gains N(0, 0.05)."""
    h, inter = cfg["hidden_size"], cfg["intermediate_size"]
    g = _gen(200 + layer, device)
    rn = lambda *s: torch.randn(*s, generator=g, device=device)                        # noqa: E731
    p = f"model.layers.{layer}."
    t = {p + "post_attention_layernorm.weight": 0.05 * rn(h), p + "mlp.gate_proj.weight": 0.02 * rn(inter, h),
         p + "mlp.up_proj.weight": 0.02 * rn(inter, h), p + "mlp.down_proj.weight": 0.02 * rn(h, inter)}
    if cfg["layer_types"][layer] == "linear_attention":
        nv, dv = cfg["linear_num_value_heads"], cfg["linear_value_head_dim"]
        a = p + "linear_attn."
        t.update({a + "in_proj_z.weight": 0.02 * rn(nv * dv, h), a + "norm.weight": 1 + 0.05 * rn(dv),
                  a + "out_proj.weight": 0.02 * rn(h, nv * dv)})
    else:
        hq, d = cfg["num_attention_heads"], cfg["head_dim"]
        a = p + "self_attn."
        t.update({a + "q_proj.weight": 0.02 * rn(2 * hq * d, h), a + "o_proj.weight": 0.02 * rn(h, hq * d),
                  a + "q_norm.weight": 0.05 * rn(d)})
    return {k: v.to(torch.bfloat16) for k, v in t.items()}


def hybrid_fill(cfg, split, n_rows, tail, device="cpu", map_noise=0.02, full=False, only=None):
    """The hybrid late-layer fill workload (dict as dense_fill's, plus layer_types); full: also each late
    layer's whole weights (hybrid_full_weights) for the exact tail; only: build these late layers alone
    (each layer's draws do not depend on the others)."""
    L, h = cfg["num_hidden_layers"], cfg["hidden_size"]
    layers = list(range(split, L)) if only is None else sorted(only)
    tensors, maps, biases = {}, {}, {}
    for l in layers:
        if cfg["layer_types"][l] == "linear_attention":
            tensors.update(gdn_layer_weights(cfg, l, device))
            g = _gen(100 + l, device)
        else:
            hkv, d = cfg["num_key_value_heads"], cfg["head_dim"]
            g = _gen(12 + l, device)
            p = f"model.layers.{l}."
            t = {p + "input_layernorm.weight": 0.05 * torch.randn(h, generator=g, device=device),
                 p + "self_attn.k_proj.weight": 0.02 * torch.randn(hkv * d, h, generator=g, device=device),
                 p + "self_attn.v_proj.weight": 0.02 * torch.randn(hkv * d, h, generator=g, device=device),
                 p + "self_attn.k_norm.weight": 0.05 * torch.randn(d, generator=g, device=device)}
            tensors.update({k: v.to(torch.bfloat16) for k, v in t.items()})
        w = torch.eye(h, device=device) + map_noise * torch.randn(h, h, generator=g, device=device) / h ** 0.5
        maps[l] = w.to(torch.bfloat16)
        biases[l] = (1e-3 * torch.randn(h, generator=g, device=device)).to(torch.bfloat16)
        if full:
            tensors.update(hybrid_full_weights(cfg, l, device))
    return dict(cfg=cfg, split=split, layers=layers, h_split=hidden_states(n_rows, h, device=device),
                P=n_rows - tail, tensors=tensors, maps=maps, biases=biases)
