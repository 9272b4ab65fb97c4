"""Oracle layer-wise forward over explicit caches (test infrastructure; see oracle/__init__.py).

Restates code/kva/model.py: Llama-3.1 (rms_norm, optional llama3 RoPE), dense Qwen3 (plus per-head
q/k RMSNorm before RoPE) and the Qwen3.5 text model (zero-centred norms, gated attention with partial
RoPE, Gated DeltaNet layers). Built from a config dict and a tensor dict with the checkpoint's
parameter names, so a transformers model's state_dict and the synthetic generators feed it alike.

Cache (code/kva/model.py:105-106, 139-159, 452-484): one dict per layer. Attention layers hold
kbuf / vbuf [Hkv, cap, d] with cap = rows + KV_RESERVE spare rows, 'n' and the views k / v = buf[:, :n];
row slot n + j receives appended row j. GDN layers hold conv [K-1, C], rec [Hv, dk, dv] fp32, len.
"""
import torch
import torch.nn.functional as F

from . import ops

KV_RESERVE = 64       # spare rows per K/V buffer (code/kva/model.py:30)
GDN_ROWS = 8192       # GDN row segment, a multiple of the 64-token chunk (code/kva/model.py:31)


class UnsupportedArchitecture(ValueError):
    """A model or model feature the forward does not implement (code/kva/model.py:35-37)."""


class OracleModel:
    def __init__(self, config, tensors, dtype=torch.float32, layers=None):
        """layers: the layer indices to load (default all); the fill of a layer needs only its own
        input norm and K / V (or GDN in-projection) weights, so partial dicts are accepted then."""
        c = config.get("text_config", config)
        self.config = c
        self.dtype = dtype
        mt = str(c.get("model_type", ""))
        if mt in ("llama", "llama_swiftkv"):
            self.arch = "llama"
        elif mt == "qwen3":
            self.arch = "qwen3"
        elif mt.startswith("qwen3_5"):
            self.arch = "qwen3_5"
        else:
            raise UnsupportedArchitecture(f"model_type {mt!r}")
        self.n_layers = c["num_hidden_layers"]
        self.hidden = c["hidden_size"]
        self.eps = c["rms_norm_eps"]
        self.n_heads = c["num_attention_heads"]
        self.n_kv = c["num_key_value_heads"]
        self.head_dim = c.get("head_dim") or self.hidden // self.n_heads
        self.scale = self.head_dim ** -0.5
        rp = c.get("rope_parameters") or c.get("rope_scaling") or {}
        theta = rp.get("rope_theta", c.get("rope_theta"))
        if self.arch == "qwen3_5":
            frac = rp.get("partial_rotary_factor", c.get("partial_rotary_factor", 1.0))
            self.rot = int(self.head_dim * frac)
            self.inv_freq = ops.inv_freq_default(theta, self.rot)
            self.layer_types = ["gdn" if t == "linear_attention" else "attn" for t in c["layer_types"]]
            self.nk, self.nv = c["linear_num_key_heads"], c["linear_num_value_heads"]
            self.dk, self.dv = c["linear_key_head_dim"], c["linear_value_head_dim"]
            self.conv_k = c["linear_conv_kernel_dim"]
        else:
            self.rot = self.head_dim
            if rp.get("rope_type") == "llama3":
                self.inv_freq = ops.inv_freq_llama3(theta, self.head_dim, rp["factor"], rp["low_freq_factor"],
                                                    rp["high_freq_factor"], rp["original_max_position_embeddings"])
            else:
                self.inv_freq = ops.inv_freq_default(theta, self.head_dim)
            self.layer_types = ["attn"] * self.n_layers
        pre = "model.language_model." if "model.language_model.embed_tokens.weight" in tensors else "model."
        t = lambda k: tensors[k].to(dtype)                 # noqa: E731
        raw = lambda k: tensors[k].float()                 # noqa: E731
        opt = lambda k: t(k) if k in tensors else None     # noqa: E731
        self.W = [None] * self.n_layers
        for i in (range(self.n_layers) if layers is None else layers):
            p = f"{pre}layers.{i}."
            w = dict(ln1=t(p + "input_layernorm.weight"), ln2=opt(p + "post_attention_layernorm.weight"),
                     gate=opt(p + "mlp.gate_proj.weight"), up=opt(p + "mlp.up_proj.weight"),
                     down=opt(p + "mlp.down_proj.weight"))
            if self.layer_types[i] == "attn":
                a = p + "self_attn."
                w.update(q=opt(a + "q_proj.weight"), k=t(a + "k_proj.weight"), v=t(a + "v_proj.weight"),
                         o=opt(a + "o_proj.weight"))
                if self.arch != "llama":
                    w.update(q_norm=opt(a + "q_norm.weight"), k_norm=t(a + "k_norm.weight"))
            else:
                a = p + "linear_attn."
                w.update(qkv=t(a + "in_proj_qkv.weight"), z=opt(a + "in_proj_z.weight"), b=t(a + "in_proj_b.weight"),
                         a=t(a + "in_proj_a.weight"), conv=t(a + "conv1d.weight").reshape(-1, self.conv_k),
                         A_log=raw(a + "A_log"), dt_bias=raw(a + "dt_bias"), norm=opt(a + "norm.weight"),
                         out=opt(a + "out_proj.weight"))
            self.W[i] = w
        self.embed_w = opt(pre + "embed_tokens.weight")
        self.norm_w = opt(pre + "norm.weight")
        self.lm_head = opt("lm_head.weight") if "lm_head.weight" in tensors else self.embed_w

    @classmethod
    def from_hf(cls, hf_model, dtype=torch.float32):
        return cls(hf_model.config.to_dict(), {k: v.detach() for k, v in hf_model.state_dict().items()}, dtype)

    # ------------------------------------------------------------------------------------- common
    def new_cache(self):
        return [dict() for _ in range(self.n_layers)]

    def embed(self, ids):
        return F.embedding(ids, self.embed_w)

    def in_norm(self, x, w):
        return (ops.rms_norm_zc if self.arch == "qwen3_5" else ops.rms_norm)(x, w, self.eps)

    def head_norm(self, x, w):
        """Per-head q/k norm: Llama's RMSNorm (Qwen3) or the zero-centred one (Qwen3.5)."""
        return self.in_norm(x, w)

    def logits(self, h):
        return F.linear(self.in_norm(h, self.norm_w), self.lm_head).float()

    def mlp(self, i, h):
        w = self.W[i]
        x = self.in_norm(h, w["ln2"])
        return h + F.linear(F.silu(F.linear(x, w["gate"])) * F.linear(x, w["up"]), w["down"])

    @staticmethod
    def append_kv(c, k, v):
        """Append rows to a layer's K/V buffers (code/kva/model.py:139-159): grow to rows + KV_RESERVE
        when full (old rows copied), write rows [n, n + m), update n and the views."""
        n = c.get("n", 0)
        m = k.shape[1]
        if c.get("kbuf") is None or n + m > c["kbuf"].shape[1]:
            cap = n + m + KV_RESERVE
            kb = k.new_empty(k.shape[0], cap, k.shape[2])
            vb = v.new_empty(v.shape[0], cap, v.shape[2])
            if n:
                kb[:, :n], vb[:, :n] = c["kbuf"][:, :n], c["vbuf"][:, :n]
            c["kbuf"], c["vbuf"] = kb, vb
        c["kbuf"][:, n:n + m] = k
        c["vbuf"][:, n:n + m] = v
        c["n"] = n + m
        c["k"], c["v"] = c["kbuf"][:, :n + m], c["vbuf"][:, :n + m]

    # ------------------------------------------------------------------------------ attention K/V
    def kv(self, i, xn, pos):
        """Post-RoPE K and V [Hkv, n, d] of normed inputs (code/kva/model.py:234-239, 340-345, 415-421)."""
        w = self.W[i]
        n = xn.shape[0]
        k = F.linear(xn, w["k"]).view(n, self.n_kv, self.head_dim)
        if self.arch != "llama":
            k = self.head_norm(k, w["k_norm"])
        v = F.linear(xn, w["v"]).view(n, self.n_kv, self.head_dim)
        cos, sin = ops.rope_cos_sin(self.inv_freq, pos, xn.dtype)
        return ops.apply_rope(k.transpose(0, 1), cos, sin), v.transpose(0, 1)

    def queries(self, i, xn, pos):
        """Post-RoPE queries [Hq, n, d] (and Qwen3.5's output gate [n, Hq * d])."""
        w = self.W[i]
        n = xn.shape[0]
        cos, sin = ops.rope_cos_sin(self.inv_freq, pos, xn.dtype)
        if self.arch == "qwen3_5":
            qg = F.linear(xn, w["q"]).view(n, self.n_heads, 2 * self.head_dim)
            q, gate = qg[..., :self.head_dim], qg[..., self.head_dim:].reshape(n, -1)
            q = self.head_norm(q, w["q_norm"]).transpose(0, 1)
            return ops.apply_rope(q, cos, sin), gate
        q = F.linear(xn, w["q"]).view(n, self.n_heads, self.head_dim)
        if self.arch == "qwen3":
            q = self.head_norm(q, w["q_norm"])
        return ops.apply_rope(q.transpose(0, 1), cos, sin), None

    def reads(self, i, x):
        """The reads of layer i's inputs x. Attention layers: pre-RoPE K and V per KV head, {'k', 'v'}:
        [tokens, Hkv, d], K head-normed for Qwen3 / Qwen3.5 (code/kva/model.py:282-287, :353-359, :558-565).
        GDN layers: the in-projection outputs that feed the state, {'q', 'k'} [tokens, nk, dk] and 'v'
        [tokens, nv, dv] before the conv, and 'ba' [tokens, 1, 2 nv] = [b | a], the beta and decay
        pre-activations (code/kva/model.py:566-571)."""
        w = self.W[i]
        xn = self.in_norm(x, w["ln1"])
        n = x.shape[0]
        if self.layer_types[i] != "attn":
            pre, b, a = self.gdn_inputs(i, xn)
            kd = self.nk * self.dk
            q, k, v = pre.split([kd, kd, self.nv * self.dv], -1)
            return dict(q=q.reshape(n, self.nk, self.dk), k=k.reshape(n, self.nk, self.dk),
                        v=v.reshape(n, self.nv, self.dv), ba=torch.cat((b, a), -1)[:, None, :])
        k = F.linear(xn, w["k"]).view(n, self.n_kv, self.head_dim)
        if self.arch != "llama":
            k = self.head_norm(k, w["k_norm"])
        return dict(k=k, v=F.linear(xn, w["v"]).view(n, self.n_kv, self.head_dim))

    def fill_kv(self, i, k, v, pos, cache):
        """Cache-only fill from given pre-RoPE K / V [tokens, Hkv, d] (code/kva/model.py:161-165)."""
        cos, sin = ops.rope_cos_sin(self.inv_freq, pos, k.dtype)
        self.append_kv(cache[i], ops.apply_rope(k.transpose(0, 1), cos, sin), v.transpose(0, 1))

    # ---------------------------------------------------------------------------------------- GDN
    def gdn_inputs(self, i, xn):
        w = self.W[i]
        return F.linear(xn, w["qkv"]), F.linear(xn, w["b"]), F.linear(xn, w["a"])

    def gdn_core(self, i, pre, b, a, cache, need_out, checkpoint_every=None, offset=0):
        """Conv + delta rule over GDN_ROWS segments continuing cache[i] (code/kva/model.py:452-484).
        Returns (out [Hv, n, dv] in pre.dtype or None, checkpoints)."""
        w, c = self.W[i], cache[i]
        n = pre.shape[0]
        kd, rep = self.nk * self.dk, self.nv // self.nk
        outs, ck = [], {}
        for r0 in range(0, n, GDN_ROWS):
            r1 = min(n, r0 + GDN_ROWS)
            m = r1 - r0
            y, c["conv"] = ops.causal_conv(pre[r0:r1], c.get("conv"), w["conv"])
            q, k, v = y.split([kd, kd, self.nv * self.dv], -1)
            q = q.reshape(m, self.nk, self.dk).float().repeat_interleave(rep, 1).transpose(0, 1)
            k = k.reshape(m, self.nk, self.dk).float().repeat_interleave(rep, 1).transpose(0, 1)
            v = v.reshape(m, self.nv, self.dv).float().transpose(0, 1)
            q = ops.l2norm(q) * self.dk ** -0.5
            k = ops.l2norm(k)
            beta = torch.sigmoid(b[r0:r1]).float().T
            g = (-w["A_log"].exp() * F.softplus(a[r0:r1].float() + w["dt_bias"])).T
            if m == 1 and not checkpoint_every:
                out, st = ops.delta_rule_recurrent(q, k, v, g, beta, c.get("rec"))
            else:
                out, st, part = ops.delta_rule(q, k, v, g, beta, c.get("rec"), checkpoint_every=checkpoint_every,
                                               offset=offset + r0, need_out=need_out)
                ck.update(part)
            c["rec"] = st
            if need_out:
                outs.append(out.to(pre.dtype))
        c["len"] = c.get("len", 0) + n
        return (torch.cat(outs, 1) if need_out else None), ck

    def gdn_mix(self, i, xn, out):
        """GDN block output from normed inputs and the delta-rule outputs (code/kva/model.py:486-499)."""
        w = self.W[i]
        n = xn.shape[0]
        z = F.linear(xn, w["z"]).view(n, self.nv, self.dv)
        y = ops.rms_norm_gated(out.transpose(0, 1), z, w["norm"], self.eps).reshape(n, -1)
        return F.linear(y, w["out"])

    # ---------------------------------------------------------------------------------- the layers
    def fill(self, i, x, pos, cache, st=None, checkpoint_every=None):
        """Cache-only fill from (predicted) layer inputs (code/kva/model.py:278-280, 510-523)."""
        xn = self.in_norm(x, self.W[i]["ln1"])
        if self.layer_types[i] == "attn":
            self.append_kv(cache[i], *self.kv(i, xn, pos))
            return {}
        pre, b, a = self.gdn_inputs(i, xn)
        _, ck = self.gdn_core(i, pre, b, a, cache, False, checkpoint_every, cache[i].get("len", 0))
        if st is not None:
            cache[i]["rec"] = cache[i]["rec"] + st.to(cache[i]["rec"])
        return ck

    def layer(self, i, h, pos, cache, gdn_checkpoint_every=None, **_):
        """Exact layer (code/kva/model.py:247-257, 436-446, 486-508)."""
        w = self.W[i]
        xn = self.in_norm(h, w["ln1"])
        if self.layer_types[i] == "attn":
            q, gate = self.queries(i, xn, pos)
            self.append_kv(cache[i], *self.kv(i, xn, pos))
            o = ops.attend(q, cache[i]["k"], cache[i]["v"], self.scale)
            if gate is not None:
                o = o * torch.sigmoid(gate)
            a = F.linear(o, w["o"])
        else:
            pre, b, ag = self.gdn_inputs(i, xn)
            out, ck = self.gdn_core(i, pre, b, ag, cache, True, gdn_checkpoint_every, cache[i].get("len", 0))
            if ck:
                cache[i].setdefault("checkpoints", {}).update(ck)
            a = self.gdn_mix(i, xn, out)
        return self.mlp(i, h + a)

    def layer_rows(self, i, h, pos, rows, cache):
        """Fill cache[i] from all rows of h, and return the exact layer output of h[rows] over that
        cache (code/kva/model.py:259-276, 525-556)."""
        w = self.W[i]
        xn = self.in_norm(h, w["ln1"])
        if self.layer_types[i] == "attn":
            self.append_kv(cache[i], *self.kv(i, xn, pos))
            q, gate = self.queries(i, xn[rows], pos[rows])
            o = ops.attend_at(q, cache[i]["k"], cache[i]["v"], self.scale, pos[rows])
            if gate is not None:
                o = o * torch.sigmoid(gate)
            hr = h[rows] + F.linear(o, w["o"])
        else:
            pre, b, a = self.gdn_inputs(i, xn)
            out, _ = self.gdn_core(i, pre, b, a, cache, True, offset=cache[i].get("len", 0))
            hr = h[rows] + self.gdn_mix(i, xn[rows], out[:, rows])
        return self.mlp(i, hr)

    def forward_exact(self, ids, hook=None, cache=None, keep=None, gdn_checkpoint_every=None):
        """Exact forward; hook(i, h) sees each layer's input (code/kva/model.py:167-181)."""
        pos = torch.arange(ids.shape[0])
        cache = self.new_cache() if cache is None else cache
        h = self.embed(ids)
        for i in range(self.n_layers):
            if hook is not None:
                hook(i, h)
            h = self.layer(i, h, pos, cache, gdn_checkpoint_every=gdn_checkpoint_every)
        if hook is not None:
            hook("final", h)
        return (self.logits(h[keep]) if keep is not None else None), cache
