"""The tiny Qwen3.5-style hybrid workload of the hybrid golden fixture (tests/golden/finish_q35.npz).

8 layers in the 3 Gated DeltaNet : 1 gated attention pattern (attention at i % 4 == 3), hidden 256, SwiGLU
512, vocab 128, eps 1e-6, fp32. GDN layers: 2 key / 4 value heads of 128, conv kernel 4. Attention layers:
4 query / 2 KV heads of head_dim 128 with the output gate, partial rotary 0.25, theta 1e7. Every weight is
a bf16-representable fp32 value (the device runs the same model in bf16); the decay parameters A_log and
dt_bias are raw fp32 as in a checkpoint. Zero-centred norm gains 0.1 N(0, 1), the GDN output norm's weight
1 + 0.1 N(0, 1), matrices N(0, 1 / fan_in).

Split 4 (late layers 4..7: GDN 4, 5, 6 and attention 7). Maps W_i = I + 0.02 N(0, 1/256) with bias
N(0, 1e-3), rounded to bf16; st corrections 0.01 N(0, 1) [4, 128, 128] for the GDN layers 4..6. Prompt
640 ids (seed 31), tail 128, keep 64; exact rows: 6 prefix rows (seed 33). Reads: one held-out document of
320 ids (seed 32).

tests/golden/make_golden.py (which runs the reference to write the fixture) and the golden tests (which run
the oracle, and the device path) build the model from this module. Every draw has its own generator.
"""
import json
from pathlib import Path

import torch

H, L, SPLIT, VOCAB, INTER = 256, 8, 4, 128, 512
NK, NV, DK, HQ, HKV, D = 2, 4, 128, 4, 2, 128
N_PROMPT, TAIL, KEEP, N_HELD, N_EXACT = 640, 128, 64, 320, 6
KINDS = ["linear_attention"] * 3 + ["full_attention"]
CONFIG = dict(model_type="qwen3_5_text", architectures=["Qwen3_5ForCausalLM"], num_hidden_layers=L,
              hidden_size=H, intermediate_size=INTER, num_attention_heads=HQ, num_key_value_heads=HKV,
              head_dim=D, vocab_size=VOCAB, rms_norm_eps=1e-6, layer_types=KINDS * 2, linear_num_key_heads=NK,
              linear_num_value_heads=NV, linear_key_head_dim=DK, linear_value_head_dim=DK,
              linear_conv_kernel_dim=4, max_position_embeddings=4096, tie_word_embeddings=False,
              torch_dtype="float32", hidden_act="silu",
              rope_parameters=dict(rope_type="default", rope_theta=1e7, partial_rotary_factor=0.25))
FIXTURE = Path(__file__).with_name("finish_q35.npz")


def _bf(t):
    return t.to(torch.bfloat16).float()


def tensors():
    """The checkpoint's tensors by their checkpoint names (fp32, CPU)."""
    g = torch.Generator().manual_seed(30)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32)            # noqa: E731
    C = 2 * NK * DK + NV * DK
    t = {"model.embed_tokens.weight": rn(VOCAB, H), "model.norm.weight": 0.1 * rn(H),
         "lm_head.weight": 0.05 * rn(VOCAB, H)}
    raw = {}
    for i, kind in enumerate(CONFIG["layer_types"]):
        p = f"model.layers.{i}."
        t.update({p + "input_layernorm.weight": 0.1 * rn(H), p + "post_attention_layernorm.weight": 0.1 * rn(H),
                  p + "mlp.gate_proj.weight": rn(INTER, H) / H ** 0.5, p + "mlp.up_proj.weight": rn(INTER, H) / H ** 0.5,
                  p + "mlp.down_proj.weight": rn(H, INTER) / INTER ** 0.5})
        if kind == "full_attention":
            a = p + "self_attn."
            t.update({a + "q_proj.weight": rn(2 * HQ * D, H) / H ** 0.5, a + "k_proj.weight": rn(HKV * D, H) / H ** 0.5,
                      a + "v_proj.weight": rn(HKV * D, H) / H ** 0.5, a + "o_proj.weight": rn(H, HQ * D) / (HQ * D) ** 0.5,
                      a + "q_norm.weight": 0.1 * rn(D), a + "k_norm.weight": 0.1 * rn(D)})
        else:
            a = p + "linear_attn."
            t.update({a + "in_proj_qkv.weight": rn(C, H) / H ** 0.5, a + "in_proj_b.weight": rn(NV, H) / H ** 0.5,
                      a + "in_proj_a.weight": 0.3 * rn(NV, H) / H ** 0.5, a + "conv1d.weight": 0.5 * rn(C, 1, 4),
                      a + "in_proj_z.weight": rn(NV * DK, H) / H ** 0.5, a + "norm.weight": 1 + 0.1 * rn(DK),
                      a + "out_proj.weight": rn(H, NV * DK) / (NV * DK) ** 0.5})
            raw[a + "A_log"] = torch.log(0.05 + 0.15 * torch.rand(NV, generator=g))
            raw[a + "dt_bias"] = 0.5 * rn(NV)
    out = {k: _bf(v).contiguous() for k, v in t.items()}
    out.update(raw)
    return out


def ids(n, seed):
    return torch.randint(0, VOCAB, (n,), generator=torch.Generator().manual_seed(seed))


def prompt_ids():
    return ids(N_PROMPT, 31)


def held_ids():
    return ids(N_HELD, 32)


def exact_rows():
    P = N_PROMPT - TAIL
    return torch.randperm(P, generator=torch.Generator().manual_seed(33))[:N_EXACT].sort().values


def maps():
    """{layer: (W [H, H], bias [H])} for late layers 4..7, bf16-representable fp32."""
    g = torch.Generator().manual_seed(34)
    out = {}
    for i in range(SPLIT, L):
        w = torch.eye(H) + 0.02 * torch.randn(H, H, generator=g) / H ** 0.5
        b = 1e-3 * torch.randn(H, generator=g)
        out[i] = (_bf(w), _bf(b))
    return out


def st():
    """{GDN layer: st [NV, DK, DK] fp32}, the terminal-state corrections of the late GDN layers."""
    g = torch.Generator().manual_seed(35)
    return {i: 0.01 * torch.randn(NV, DK, DK, generator=g) for i in range(SPLIT, L) if i % 4 != 3}


def probes(seed, *shape):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def write_checkpoint(path):
    """config.json + model.safetensors in the checkpoint layout the reference loader reads."""
    from safetensors.torch import save_file
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(CONFIG))
    save_file(tensors(), str(path / "model.safetensors"))
    return path


def read_arrays(tag, reads):
    """One layer's reads {name: [n, heads, width]} as projections of each head vector onto 4 probes, plus
    their full first and last rows."""
    out = {}
    for r, t in sorted(reads.items()):
        t = t.double()
        out[f"{tag}_{r}_u"] = (t @ probes(200 + t.shape[-1], t.shape[-1], 4)).numpy()
        out[f"{tag}_{r}_ends"] = t[[0, -1]].numpy()
    return out


def cosine_score(pred, true):
    """One document's read score of one layer as the held-out selection forms it (code/scripts/fit_sweep.py:
    307-313): per read, the mean over rows and heads of the cosine over the head vector, then the mean over
    the reads."""
    import torch.nn.functional as F
    return sum(F.cosine_similarity(pred[r].float(), true[r].float(), dim=-1).mean().item() for r in true) / len(true)


def slots(P, n):
    """The cache slots kept in full: 0, 1 and P - 1, then P and the last one when the cache holds the tail."""
    return [0, 1, P - 1] + ([P, n - 1] if n > P else [])


def cache_arrays(tag, cache, P, types):
    """The late layers' caches: attention K / V as probe projections [Hkv, n] plus the slots of slots();
    GDN recurrent states [NV, DK, DK] as probe projections plus 4 rows of head 0, and the conv states in full."""
    import numpy as np
    u_d = probes(102, D)
    out = {}
    for i in range(SPLIT, L):
        c = cache[i]
        if not c:
            out[f"{tag}_dropped_{i}"] = np.array(1)
            continue
        if types[i] == "attn":
            out[f"{tag}_n_{i}"] = np.array(c["n"])
            for part in ("k", "v"):
                t = c[part].double()
                n = t.shape[1]
                out[f"{tag}_{part}_u_{i}"] = (t @ u_d).numpy()
                out[f"{tag}_{part}_rows_{i}"] = t[:, slots(P, n)].numpy()
        else:
            rec = c["rec"].double()
            out[f"{tag}_rec_u_{i}"] = (rec @ probes(104, DK)).numpy()
            out[f"{tag}_rec_h0_{i}"] = rec[0, :4].numpy()
            out[f"{tag}_conv_{i}"] = c["conv"].double().numpy()
    return out
