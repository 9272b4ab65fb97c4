"""Device-side fill model: the per-layer fill API of code/kva/model.py over explicit caches, with the
arithmetic in librfill's HIP kernels.

  fill(i, x, pos, cache)        cache-only fill from (predicted) layer inputs x [P, H] bf16
                                (code/kva/model.py:278-280, 510-523)
  fill_kv(i, k, v, pos, cache)  cache-only fill from given pre-RoPE K / V [P, Hkv, d]
                                (code/kva/model.py:161-165)
  new_cache()                   one dict per layer (code/kva/model.py:105-106)

Cache layout (code/kva/model.py:139-159): attention layers hold kbuf / vbuf [Hkv, cap, d] bf16 with
cap = rows + KV_RESERVE, 'n' and the views k / v = buf[:, :n]; appended row j lands in slot n + j.
The kernels write straight into the buffer; growing it (allocate rows + KV_RESERVE, copy the old rows)
is the only host-side step and happens before the launch.

Packed weights, built once per layer at load: wkv = [W_k; W_v] with the input-norm gain folded into
its columns (rf_fold_norm), the k_norm gain, and the RoPE frequencies on the device.
"""
import torch

from . import ops
from ._lib import UnsupportedArchitecture

KV_RESERVE = 64


class FillModel:
    def __init__(self, config, tensors, device="cuda", layers=None):
        c = config.get("text_config", config)
        mt = str(c.get("model_type", ""))
        if mt in ("llama", "llama_swiftkv"):
            self.arch = "llama"
        elif mt == "qwen3":
            self.arch = "qwen3"
        elif mt.startswith("qwen3_5"):
            self.arch = "qwen3_5"
        else:
            raise UnsupportedArchitecture(f"model_type {mt!r} (llama, llama_swiftkv, qwen3, qwen3_5)")
        self.device = torch.device(device)
        self.n_layers = c["num_hidden_layers"]
        self.hidden = c["hidden_size"]
        self.eps = float(c["rms_norm_eps"])
        self.n_heads = c["num_attention_heads"]
        self.n_kv = c["num_key_value_heads"]
        self.head_dim = c.get("head_dim") or self.hidden // self.n_heads
        rp = c.get("rope_parameters") or c.get("rope_scaling") or {}
        theta = rp.get("rope_theta", c.get("rope_theta"))
        if self.arch == "qwen3_5":
            frac = rp.get("partial_rotary_factor", c.get("partial_rotary_factor", 1.0))
            self.rot = int(self.head_dim * frac)
            inv = ops.inv_freq_default(theta, self.rot)
            self.layer_types = ["gdn" if t == "linear_attention" else "attn" for t in c["layer_types"]]
        else:
            if self.arch == "qwen3" and rp.get("rope_type", "default") != "default":
                raise UnsupportedArchitecture(f"Qwen3 rope_type {rp.get('rope_type')!r}")
            self.rot = self.head_dim
            if rp.get("rope_type") == "llama3":
                inv = ops.inv_freq_llama3(theta, self.head_dim, rp["factor"], rp["low_freq_factor"],
                                          rp["high_freq_factor"], rp["original_max_position_embeddings"])
            else:
                inv = ops.inv_freq_default(theta, self.head_dim)
            self.layer_types = ["attn"] * self.n_layers
        self.inv_freq = inv.to(self.device)
        self.knorm_kind = 1 if self.arch == "qwen3_5" else 0
        pre = "model.language_model." if "model.language_model.embed_tokens.weight" in tensors else "model."
        want = range(self.n_layers) if layers is None else layers
        self.W = [None] * self.n_layers
        for i in want:
            self.W[i] = self._pack(i, f"{pre}layers.{i}.", tensors)

    def _pack(self, i, p, tensors):
        dev = lambda k: tensors[k].to(self.device, torch.bfloat16).contiguous()   # noqa: E731
        if self.layer_types[i] != "attn":
            return dict(kind="gdn")
        a = p + "self_attn."
        ln1 = dev(p + "input_layernorm.weight")
        wkv = torch.cat((dev(a + "k_proj.weight"), dev(a + "v_proj.weight")), 0)
        w = dict(kind="attn", ln1=ln1, wkv=ops.fold_norm(wkv, ln1, self.knorm_kind))
        if self.arch != "llama":
            w["k_norm"] = dev(a + "k_norm.weight")
        return w

    @classmethod
    def from_hf(cls, hf_model, device="cuda", layers=None):
        return cls(hf_model.config.to_dict(), {k: v.detach() for k, v in hf_model.state_dict().items()}, device,
                   layers)

    def new_cache(self):
        return [dict() for _ in range(self.n_layers)]

    def rope_table(self, pos):
        """The [P, rot] cos / sin table of positions pos (one table serves every late layer)."""
        return ops.rope_table(pos.to(self.device, torch.int64), self.inv_freq)

    @staticmethod
    def reserve(c, m, hkv, d, device):
        """Make room for m more rows in cache dict c (code/kva/model.py:145-155: grow to n + m +
        KV_RESERVE, copy the old rows); returns the first slot to write."""
        n = c.get("n", 0)
        if c.get("kbuf") is None or n + m > c["kbuf"].shape[1]:
            cap = n + m + KV_RESERVE
            kb = torch.empty(hkv, cap, d, dtype=torch.bfloat16, device=device)
            vb = torch.empty(hkv, cap, d, dtype=torch.bfloat16, device=device)
            if n:
                kb[:, :n].copy_(c["kbuf"][:, :n])
                vb[:, :n].copy_(c["vbuf"][:, :n])
            c["kbuf"], c["vbuf"] = kb, vb
        return n

    @staticmethod
    def commit(c, m):
        n = c.get("n", 0) + m
        c["n"] = n
        c["k"], c["v"] = c["kbuf"][:, :n], c["vbuf"][:, :n]

    def _layer(self, i):
        w = self.W[i]
        if w is None:
            raise ValueError(f"layer {i} was not packed (FillModel(layers=...))")
        if w["kind"] != "attn":
            raise UnsupportedArchitecture(f"layer {i}: Gated DeltaNet fill is not built in this library version")
        return w

    def fill(self, i, x, pos, cache, st=None, ssq=None, cs=None):
        """Cache-only fill of layer i from inputs x [P, H] bf16 at positions pos. ssq: x's row
        sum-of-squares partials if already known (rf_map_apply / rf_row_scatter produce them);
        cs: the RoPE table of pos if already built."""
        w = self._layer(i)
        if st is not None:
            raise ValueError("st corrects GDN recurrent states; layer is attention")
        P = x.shape[0]
        if ssq is None:
            ssq = ops.row_ssq(x)
        if cs is None:
            cs = self.rope_table(pos)
        c = cache[i]
        slot = self.reserve(c, P, self.n_kv, self.head_dim, x.device)
        ops.norm_kv_write(x, ssq, self.eps, w["wkv"], self.n_kv, self.head_dim, w.get("k_norm"), self.knorm_kind,
                          cs, c["kbuf"], c["vbuf"], slot)
        self.commit(c, P)
        return {}

    def fill_kv(self, i, k, v, pos, cache, cs=None):
        """Cache-only fill from pre-RoPE K and V [P, Hkv, d] (the reads() layout)."""
        self._layer(i)
        P = k.shape[0]
        if cs is None:
            cs = self.rope_table(pos)
        c = cache[i]
        slot = self.reserve(c, P, self.n_kv, self.head_dim, k.device)
        ops.rope_kv_write(k, v, cs, c["kbuf"], c["vbuf"], slot)
        self.commit(c, P)
