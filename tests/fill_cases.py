"""Random small models in the checkpoint's parameter naming, shared by the fill parity tests, so that the
oracle (CPU) and the device fill model are built from the very same tensors."""
import torch


def rel_err(a, b):
    """Relative Frobenius error |a - b| / |b| in fp64."""
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


def attn_config(arch, hidden, hkv, d, theta, n_heads=None, rope=None, eps=1e-5, layers=1, rot_frac=None):
    n_heads = n_heads or 2 * hkv
    c = dict(model_type={"llama": "llama", "qwen3": "qwen3", "qwen3_5": "qwen3_5_text"}[arch],
             num_hidden_layers=layers, hidden_size=hidden, num_attention_heads=n_heads, num_key_value_heads=hkv,
             head_dim=d, rms_norm_eps=eps, intermediate_size=256)
    if arch == "qwen3_5":
        c.update(layer_types=["full_attention"] * layers, linear_num_key_heads=2, linear_num_value_heads=4,
                 linear_key_head_dim=16, linear_value_head_dim=16, linear_conv_kernel_dim=4,
                 rope_parameters=dict(rope_type="default", rope_theta=theta, partial_rotary_factor=rot_frac or 1.0))
    elif rope is not None:
        c["rope_scaling"] = dict(rope, rope_theta=theta)
    else:
        c["rope_theta"] = theta
    return c


def random_tensors(cfg, seed=0, vocab=64):
    """Every parameter an attention-only model of cfg needs (HF names), fp32, seeded."""
    g = torch.Generator().manual_seed(seed)
    h, hkv, d, hq, inter = (cfg["hidden_size"], cfg["num_key_value_heads"], cfg["head_dim"],
                            cfg["num_attention_heads"], cfg["intermediate_size"])
    qw = 2 * hq * d if cfg["model_type"].startswith("qwen3_5") else hq * d
    t = {"model.embed_tokens.weight": torch.randn(vocab, h, generator=g),
         "model.norm.weight": 1 + 0.1 * torch.randn(h, generator=g),
         "lm_head.weight": 0.05 * torch.randn(vocab, h, generator=g)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        t.update({p + "input_layernorm.weight": 1 + 0.1 * torch.randn(h, generator=g),
                  p + "post_attention_layernorm.weight": 1 + 0.1 * torch.randn(h, generator=g),
                  p + "self_attn.q_proj.weight": torch.randn(qw, h, generator=g) / h ** 0.5,
                  p + "self_attn.k_proj.weight": torch.randn(hkv * d, h, generator=g) / h ** 0.5,
                  p + "self_attn.v_proj.weight": torch.randn(hkv * d, h, generator=g) / h ** 0.5,
                  p + "self_attn.o_proj.weight": torch.randn(h, hq * d, generator=g) / (hq * d) ** 0.5,
                  p + "mlp.gate_proj.weight": torch.randn(inter, h, generator=g) / h ** 0.5,
                  p + "mlp.up_proj.weight": torch.randn(inter, h, generator=g) / h ** 0.5,
                  p + "mlp.down_proj.weight": torch.randn(h, inter, generator=g) / inter ** 0.5})
        if cfg["model_type"] != "llama":
            t[p + "self_attn.q_norm.weight"] = 1 + 0.1 * torch.randn(d, generator=g)
            t[p + "self_attn.k_norm.weight"] = 1 + 0.1 * torch.randn(d, generator=g)
    return {k: v.to(torch.bfloat16) for k, v in t.items()}


def inputs(n, h, seed=1, outliers=True):
    """Layer inputs with a spread of channel scales and a few outlier channels (bf16)."""
    g = torch.Generator().manual_seed(seed)
    gain = torch.exp(0.5 * torch.randn(h, generator=g))
    if outliers:
        gain[torch.randperm(h, generator=g)[:4]] *= 20
    return (torch.randn(n, h, generator=g) * gain).to(torch.bfloat16)


# name -> (arch, hidden, kv heads, head dim, theta, extra config kwargs)
CASES = {
    "llama_c1": ("llama", 256, 2, 64, 1e4, {}),
    "llama3_scaled": ("llama", 512, 4, 128, 5e5, dict(rope=dict(rope_type="llama3", factor=8.0, low_freq_factor=1.0,
                                                                high_freq_factor=4.0,
                                                                original_max_position_embeddings=256))),
    "qwen3_knorm": ("qwen3", 512, 2, 128, 1e6, dict(eps=1e-6)),
    "qwen35_attn": ("qwen3_5", 2048, 2, 256, 1e7, dict(eps=1e-6, rot_frac=0.25)),
}


def case(name, layers=1, seed=0):
    arch, h, hkv, d, theta, kw = CASES[name]
    cfg = attn_config(arch, h, hkv, d, theta, layers=layers, **kw)
    return cfg, random_tensors(cfg, seed)


def gdn_config(hidden=512, nk=2, nv=4, layers=1, eps=1e-6):
    """A Qwen3.5 text config whose layers are all Gated DeltaNet (dk = dv = 128, conv kernel 4)."""
    return dict(model_type="qwen3_5_text", num_hidden_layers=layers, hidden_size=hidden, num_attention_heads=4,
                num_key_value_heads=2, head_dim=128, rms_norm_eps=eps, intermediate_size=256,
                layer_types=["linear_attention"] * layers, linear_num_key_heads=nk, linear_num_value_heads=nv,
                linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4,
                rope_parameters=dict(rope_type="default", rope_theta=1e7, partial_rotary_factor=0.25))


def gdn_tensors(cfg, seed=0):
    """GDN layer weights (checkpoint names). Gates: A_log = log U(0.05, 0.2), dt_bias N(0, 0.5), W_a small,
    so decays stay mild and the state integrates many rows."""
    g = torch.Generator().manual_seed(seed)
    h, nk, nv = cfg["hidden_size"], cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    C = 2 * nk * 128 + nv * 128
    t = {}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        a = p + "linear_attn."
        t.update({p + "input_layernorm.weight": 0.1 * torch.randn(h, generator=g),
                  a + "in_proj_qkv.weight": torch.randn(C, h, generator=g) / h ** 0.5,
                  a + "in_proj_b.weight": torch.randn(nv, h, generator=g) / h ** 0.5,
                  a + "in_proj_a.weight": 0.3 * torch.randn(nv, h, generator=g) / h ** 0.5,
                  a + "conv1d.weight": 0.5 * torch.randn(C, 1, 4, generator=g)})
        t = {k: v.to(torch.bfloat16) for k, v in t.items()}
        t[a + "A_log"] = torch.log(0.05 + 0.15 * torch.rand(nv, generator=g))
        t[a + "dt_bias"] = 0.5 * torch.randn(nv, generator=g)
    return t


def hybrid_config(layer_types, hidden=512, nk=2, nv=4, hkv=2, d=128, eps=1e-6):
    """A Qwen3.5 text config with the given layer kinds ("gdn" / "attn"): GDN heads as gdn_config, gated
    attention with 2 hkv query heads of head_dim d, partial rotary 0.25."""
    c = gdn_config(hidden, nk, nv, len(layer_types), eps)
    c.update(layer_types=["linear_attention" if t == "gdn" else "full_attention" for t in layer_types],
             num_key_value_heads=hkv, num_attention_heads=2 * hkv, head_dim=d)
    return c


def hybrid_tensors(cfg, seed=0, vocab=64):
    """Every parameter of a whole Qwen3.5 model of cfg (checkpoint names): zero-centred norm gains
    0.1 N(0, 1), the GDN output norm's weight 1 + 0.1 N(0, 1), gates as gdn_tensors, matrices N(0, 1/fan_in)."""
    g = torch.Generator().manual_seed(seed)
    h, hkv, d, hq, inter = (cfg["hidden_size"], cfg["num_key_value_heads"], cfg["head_dim"],
                            cfg["num_attention_heads"], cfg["intermediate_size"])
    nk, nv = cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    C = 2 * nk * 128 + nv * 128
    rn = lambda *s: torch.randn(*s, generator=g)                                   # noqa: E731
    t = {"model.embed_tokens.weight": rn(vocab, h), "model.norm.weight": 0.1 * rn(h),
         "lm_head.weight": 0.05 * rn(vocab, h)}
    raw = {}
    for i, kind in enumerate(cfg["layer_types"]):
        p = f"model.layers.{i}."
        t.update({p + "input_layernorm.weight": 0.1 * rn(h), p + "post_attention_layernorm.weight": 0.1 * rn(h),
                  p + "mlp.gate_proj.weight": rn(inter, h) / h ** 0.5, p + "mlp.up_proj.weight": rn(inter, h) / h ** 0.5,
                  p + "mlp.down_proj.weight": rn(h, inter) / inter ** 0.5})
        if kind == "full_attention":
            a = p + "self_attn."
            t.update({a + "q_proj.weight": rn(2 * hq * d, h) / h ** 0.5, a + "k_proj.weight": rn(hkv * d, h) / h ** 0.5,
                      a + "v_proj.weight": rn(hkv * d, h) / h ** 0.5, a + "o_proj.weight": rn(h, hq * d) / (hq * d) ** 0.5,
                      a + "q_norm.weight": 0.1 * rn(d), a + "k_norm.weight": 0.1 * rn(d)})
        else:
            a = p + "linear_attn."
            t.update({a + "in_proj_qkv.weight": rn(C, h) / h ** 0.5, a + "in_proj_b.weight": rn(nv, h) / h ** 0.5,
                      a + "in_proj_a.weight": 0.3 * rn(nv, h) / h ** 0.5, a + "conv1d.weight": 0.5 * rn(C, 1, 4),
                      a + "in_proj_z.weight": rn(nv * 128, h) / h ** 0.5, a + "norm.weight": 1 + 0.1 * rn(128),
                      a + "out_proj.weight": rn(h, nv * 128) / (nv * 128) ** 0.5})
            raw[a + "A_log"] = torch.log(0.05 + 0.15 * torch.rand(nv, generator=g))
            raw[a + "dt_bias"] = 0.5 * rn(nv)
    out = {k: v.to(torch.bfloat16) for k, v in t.items()}
    out.update(raw)
    return out
