"""The tiny Llama-style workload of the golden fixtures: 8 layers, hidden 256, 4 query / 2 KV heads,
head_dim 64, SwiGLU 688, vocab 1024, RoPE theta 1e4, fp32; matrices N(0, 0.02) from seed 0, norm
gains 1. Split 5 (late layers 5..7), maps fitted from one 4096-token calibration document (uniform ids,
seed 1) with lambda = 1e-2 (times the centred scatter's mean diagonal); prompt 2048 ids (seed 2), exact
tail 256, keep 256; the exact-row variant marks 18 prefix rows (1 % of P = 1792, seed 3) exact.

Both tests/golden/make_golden.py (which runs the reference implementation to write the fixture) and
the golden tests (which run the oracle and the device path) build the model from this module, so they
see the same weights and inputs. Every random draw uses its own torch.Generator on the CPU.
"""
import json
from pathlib import Path

import torch

CONFIG = dict(model_type="llama", architectures=["LlamaForCausalLM"], num_hidden_layers=8, hidden_size=256,
              intermediate_size=688, num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=1024,
              rms_norm_eps=1e-5, rope_theta=10000.0, rope_scaling=None, max_position_embeddings=4096,
              tie_word_embeddings=False, torch_dtype="float32", hidden_act="silu", attention_bias=False)
SPLIT, N_CAL, N_PROMPT, TAIL, KEEP, LAM = 5, 4096, 2048, 256, 256, 1e-2
N_EXACT = 18
CAL_DOCS2 = ((300, 10), (260, 11))      # the two-document capture that pins the shift convention
FIXTURE = Path(__file__).with_name("finish_c1.npz")


def tensors():
    """The checkpoint's tensors by their checkpoint names (fp32, CPU)."""
    c = CONFIG
    H, I, V, L = c["hidden_size"], c["intermediate_size"], c["vocab_size"], c["num_hidden_layers"]
    q, kv = c["num_attention_heads"] * c["head_dim"], c["num_key_value_heads"] * c["head_dim"]
    g = torch.Generator().manual_seed(0)
    mat = lambda r, k: (0.02 * torch.randn(r, k, generator=g, dtype=torch.float32)).contiguous()   # noqa: E731
    out = {"model.embed_tokens.weight": mat(V, H)}
    for i in range(L):
        p = f"model.layers.{i}."
        out[p + "input_layernorm.weight"] = torch.ones(H)
        out[p + "post_attention_layernorm.weight"] = torch.ones(H)
        out[p + "self_attn.q_proj.weight"] = mat(q, H)
        out[p + "self_attn.k_proj.weight"] = mat(kv, H)
        out[p + "self_attn.v_proj.weight"] = mat(kv, H)
        out[p + "self_attn.o_proj.weight"] = mat(H, q)
        out[p + "mlp.gate_proj.weight"] = mat(I, H)
        out[p + "mlp.up_proj.weight"] = mat(I, H)
        out[p + "mlp.down_proj.weight"] = mat(H, I)
    out["model.norm.weight"] = torch.ones(H)
    out["lm_head.weight"] = mat(V, H)
    return out


def ids(n, seed):
    return torch.randint(0, CONFIG["vocab_size"], (n,), generator=torch.Generator().manual_seed(seed))


def calibration_ids():
    return ids(N_CAL, 1)


def two_documents():
    return [ids(n, seed) for n, seed in CAL_DOCS2]


def prompt_ids():
    return ids(N_PROMPT, 2)


def exact_rows():
    P = N_PROMPT - TAIL
    g = torch.Generator().manual_seed(3)
    return torch.randperm(P, generator=g)[:N_EXACT].sort().values


def probes(seed, *shape):
    """Fixed random probe vectors: the fixture stores projections of large outputs onto them."""
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def write_checkpoint(path):
    """config.json + model.safetensors in the checkpoint layout the reference loader reads."""
    from safetensors.torch import save_file
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(CONFIG))
    save_file(tensors(), str(path / "model.safetensors"))
    return path


def state_arrays(state, tag=""):
    """A capture state's sums: shifts and first sums in full, the scatters as probe projections."""
    import numpy as np
    u_h, v_h = probes(100, 256), probes(101, 256)
    out = {f"{tag}n": np.array(state["n"]), f"{tag}cx": state["cx"].double().numpy(),
           f"{tag}sx": state["sx"].double().numpy(), f"{tag}sxx_u": (state["sxx"].double() @ u_h).numpy(),
           f"{tag}sxx_diag": state["sxx"].double().diagonal().numpy()}
    for i in sorted(state["layers"]):
        out[f"{tag}cy_{i}"] = state["cy"][i].double().numpy()
        out[f"{tag}sy_{i}"] = state["sy"][i].double().numpy()
        out[f"{tag}sxy_u_{i}"] = (state["sxy"][i].double() @ u_h).numpy()
        out[f"{tag}sxy_tv_{i}"] = (state["sxy"][i].double().T @ v_h).numpy()
    return out


def summarise(state, state2, maps, runs):
    """The fixture's arrays (numpy, float64 unless noted) from the capture states of split 5 (one
    4096-token document; and the two-document capture, keys prefixed 'two_'), the fitted maps
    {i: (W [d_out, d_in], bias)} and the finish runs {name: (logits, cache, P, row_inputs)}.
    Large tensors are kept as projections onto probe vectors plus a few full slices."""
    import numpy as np
    u_h = probes(100, 256)
    v_h = probes(101, 256)
    u_d = probes(102, 64)
    u_v = probes(103, 1024, 4)
    out = state_arrays(state)
    out.update(state_arrays(state2, "two_"))
    for i, (w, b) in sorted(maps.items()):
        out[f"w_u_{i}"] = (w.double() @ u_h).numpy()
        out[f"w_tv_{i}"] = (w.double().T @ v_h).numpy()
        out[f"w_row0_{i}"] = w[0].double().numpy()
        out[f"bias_{i}"] = b.double().numpy()
    for name, (logits, cache, P, row_inputs) in runs.items():
        out[f"{name}_P"] = np.array(P)
        lg = logits.double()
        out[f"{name}_logits_u"] = (lg @ u_v).numpy()
        out[f"{name}_logits_last"] = lg[-1].numpy()
        out[f"{name}_argmax"] = lg.argmax(-1).numpy()
        for i in range(SPLIT, CONFIG["num_hidden_layers"]):
            c = cache[i]
            out[f"{name}_n_{i}"] = np.array(c["n"])
            for part in ("k", "v"):
                t = c[part].double()                                  # [Hkv, n, d]
                out[f"{name}_{part}_u_{i}"] = (t @ u_d).float().numpy()   # [Hkv, n]
                out[f"{name}_{part}_rows_{i}"] = t[:, [0, 1, P - 1, P, t.shape[1] - 1]].numpy()
            if row_inputs:
                out[f"{name}_hr_{i}"] = row_inputs[i].double().numpy()
    return out


# ---- the map file fixture (Projector.save / load, code/kva/kva.py:161-193)

PROJ_FIXTURE = Path(__file__).with_name("projector_ref.safetensors")
PROJ_SPLIT = 3
PROJ_META = {"fit": "golden", "lam": 0.01, "layers": "3,4", "n": 4096}


def projector_tensors():
    """The fixture projector's maps {layer: (W [24, 40] fp32, bias [24] fp32)} for late layers 3 and 4 of a
    5-layer stack: seeded normals at a few scales, so the bf16 cast in save() rounds most entries, plus
    entries that pin the cast (an exact bf16 value, a round-to-nearest-even tie, -0.0) and the |w| <= 1e4
    limit (1e4 itself, which save() and load() accept)."""
    g = torch.Generator().manual_seed(40)
    out = {}
    for L, s in ((3, 0.05), (4, 3.0)):
        w = s * torch.randn(24, 40, generator=g, dtype=torch.float32)
        b = 1e-3 * torch.randn(24, generator=g, dtype=torch.float32)
        w[0, 0] = 1.5                      # exact in bf16
        w[0, 1] = 1.0 + 2.0 ** -8          # tie between 1 and 1 + 2^-7: rounds to the even pattern, 1.0
        w[0, 2] = 1.0 + 3 * 2.0 ** -8      # tie between 1 + 2^-7 and 1 + 2^-6: rounds to 1 + 2^-6
        w[0, 3] = -0.0
        w[1, 0] = 1e4
        out[L] = (w, b)
    return out
