"""Device-side fill model: the per-layer fill API of code/kva/model.py over explicit caches, with the
arithmetic in librfill's HIP kernels.

  fill(i, x, pos, cache)        cache-only fill from (predicted) layer inputs x [P, H] bf16
                                (code/kva/model.py:278-280, 510-523)
  fill_kv(i, k, v, pos, cache)  cache-only fill from given pre-RoPE K / V [P, Hkv, d]
                                (code/kva/model.py:161-165)
  forward_exact(ids, hook)      exact forward of one document, hook(i, h) on every layer input
                                (code/kva/model.py:167-181)
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
GDN_ROWS = 8192          # rows per GDN workspace pass (the reference's GDN segment, code/kva/model.py:31)
# rows per pass when GDN layers fill together (rf_gdn_fill_batch): a 32K prompt's rows in one pass. The passes
# carry the state exactly, so this changes no result; the Qwen3.5-shaped 32K hybrid fill measured 28.33 ms in
# one pass against 28.65 ms in two and 28.92 ms in 8192-row passes (same box, bit-identical states). A single
# layer keeps 8192-row workspaces: it runs half of one per pass, the next pass's prep beside the current scan.
GDN_BATCH_ROWS = 32768


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
            self.nk, self.nv = c.get("linear_num_key_heads"), c.get("linear_num_value_heads")
            self.dk, self.dv = c.get("linear_key_head_dim"), c.get("linear_value_head_dim")
            self.conv_k = c.get("linear_conv_kernel_dim")
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
        self._src, self._pre = tensors, pre                # the full-layer weights are packed on first use
        self.scale = self.head_dim ** -0.5
        want = range(self.n_layers) if layers is None else layers
        self.W = [None] * self.n_layers
        self._gdn_ws = None
        for i in want:
            self.W[i] = self._pack(i, f"{pre}layers.{i}.", tensors)

    def _pack(self, i, p, tensors):
        dev = lambda k: tensors[k].to(self.device, torch.bfloat16).contiguous()   # noqa: E731
        if self.layer_types[i] != "attn":
            return self._pack_gdn(p, tensors, dev)
        a = p + "self_attn."
        ln1 = dev(p + "input_layernorm.weight")
        wkv = torch.cat((dev(a + "k_proj.weight"), dev(a + "v_proj.weight")), 0)
        w = dict(kind="attn", ln1=ln1, wkv=ops.fold_norm(wkv, ln1, self.knorm_kind))
        if self.arch != "llama":
            w["k_norm"] = dev(a + "k_norm.weight")
        return w

    def _pack_gdn(self, p, tensors, dev):
        """GDN layer: in-projections [W_qkv; W_b; W_a] with the zero-centred input norm's (1 + g) folded
        into the columns, zero rows up to a multiple of 256; conv weight [C, 4]; the gates' A_log and
        dt_bias in fp32 as stored (code/kva/model.py:396-400)."""
        if self.conv_k != 4 or self.dk != 128 or self.dv != 128:
            raise UnsupportedArchitecture(f"GDN conv kernel {self.conv_k}, head dims {self.dk} / {self.dv} "
                                          f"(kernels: 4, 128 / 128)")
        a = p + "linear_attn."
        ln1 = dev(p + "input_layernorm.weight")
        w_in = torch.cat((dev(a + "in_proj_qkv.weight"), dev(a + "in_proj_b.weight"), dev(a + "in_proj_a.weight")), 0)
        n = w_in.shape[0]
        pad = (-n) % 256
        if pad:
            w_in = torch.cat((w_in, w_in.new_zeros(pad, w_in.shape[1])), 0)
        conv = tensors[a + "conv1d.weight"].to(self.device, torch.bfloat16).reshape(-1, self.conv_k).contiguous()
        return dict(kind="gdn", ln1=ln1, w_in=ops.fold_norm(w_in, ln1, 1), conv=conv,
                    a_log=tensors[a + "A_log"].to(self.device, torch.float32).contiguous(),
                    dt_bias=tensors[a + "dt_bias"].to(self.device, torch.float32).contiguous())

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
    def reserve(c, m, hkv, d, device, fresh=False):
        """Make room for m more rows in cache dict c (code/kva/model.py:145-155: grow to n + m +
        KV_RESERVE, copy the old rows); returns the first slot to write. fresh: new buffers even when the
        old ones have room (c shares its buffers with another cache dict that must not see the new rows)."""
        n = c.get("n", 0)
        if c.get("kbuf") is None or n + m > c["kbuf"].shape[1] or fresh:
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

    def _layer(self, i, kind="attn"):
        w = self.W[i]
        if w is None:
            raise ValueError(f"layer {i} was not packed (FillModel(layers=...))")
        if w["kind"] != kind:
            raise ValueError(f"layer {i} is a {w['kind']} layer")
        return w

    def fill(self, i, x, pos, cache, st=None, ssq=None, cs=None, checkpoint_every=None):
        """Cache-only fill of layer i from inputs x [P, H] bf16 at positions pos (code/kva/model.py:
        278-280, 510-523). Attention layers: K / V into the cache. GDN layers: conv state and recurrent
        state continued over the rows, then + st (the terminal-state correction) if given. ssq: x's row
        sum-of-squares partials if already known (rf_map_apply / rf_row_scatter produce them); cs: the
        RoPE table of pos if already built."""
        if self.layer_types[i] == "gdn":
            return self._fill_gdn(i, x, cache, st, ssq, checkpoint_every)
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
                          cs, c["kbuf"], c["vbuf"], slot,
                          workspace=self.gemm_workspace(P, w["wkv"].shape[0], x.shape[1], x.device))
        self.commit(c, P)
        return {}

    def fill_attn_batch(self, ids, xs, pos, cache, ssqs=None, cs=None):
        """fill() of several attention layers over the same rows at once (ops.norm_kv_write_batch): every
        layer's K / V bit-identical to its fill() without a split-K workspace. Layers whose caches do not take
        the rows at one slot in one buffer layout are filled one at a time."""
        ids = list(ids)
        if any(self.layer_types[i] != "attn" for i in ids):
            raise ValueError(f"fill_attn_batch: attention layers only, got {ids}")
        P = xs[0].shape[0]
        if P == 0:
            return
        ssqs = [ops.row_ssq(x) if q is None else q for x, q in zip(xs, ssqs or [None] * len(ids))]
        if cs is None:
            cs = self.rope_table(pos)
        slots = [self.reserve(cache[i], P, self.n_kv, self.head_dim, xs[0].device) for i in ids]
        c0 = cache[ids[0]]
        same = all(s == slots[0] and cache[i]["kbuf"].shape == c0["kbuf"].shape
                   and cache[i]["kbuf"].stride() == c0["kbuf"].stride() for i, s in zip(ids, slots))
        if not same or len(ids) > ops.MAP_BATCH_MAX:
            for i, x, q, s in zip(ids, xs, ssqs, slots):
                w, c = self._layer(i), cache[i]
                ops.norm_kv_write(x, q, self.eps, w["wkv"], self.n_kv, self.head_dim, w.get("k_norm"),
                                  self.knorm_kind, cs, c["kbuf"], c["vbuf"], s,
                                  workspace=self.gemm_workspace(P, w["wkv"].shape[0], x.shape[1], x.device))
        else:
            ws = [self._layer(i) for i in ids]
            ops.norm_kv_write_batch(xs, ssqs, self.eps, [w["wkv"] for w in ws], self.n_kv, self.head_dim,
                                    [w.get("k_norm") for w in ws], self.knorm_kind, cs,
                                    [cache[i]["kbuf"] for i in ids], [cache[i]["vbuf"] for i in ids], slots[0])
        for i in ids:
            self.commit(cache[i], P)

    def _fill_gdn(self, i, x, cache, st, ssq, checkpoint_every):
        """checkpoint_every (a multiple of the 64-row chunk): also return {len + t: state after t rows} for
        every t (rows of this call) that is a multiple of it (code/kva/ops.py:206-209, :258-260). The rows
        then go through the kernels in segments of that many rows; a segment boundary on the chunk grid
        leaves every chunk's arithmetic, and so the final state, unchanged."""
        if checkpoint_every and (checkpoint_every <= 0 or checkpoint_every % 64):
            raise ValueError(f"checkpoint_every {checkpoint_every}: a positive multiple of the 64-row chunk")
        w = self._layer(i, "gdn")
        P = x.shape[0]
        c = cache[i]
        if P == 0:
            return {}
        if ssq is None:
            ssq = ops.row_ssq(x)
        pre = self._fill_rows(w, x, ssq)
        rec = c.get("rec")
        rec = (torch.zeros(self.nv, self.dk, self.dv, dtype=torch.float32, device=x.device) if rec is None
               else rec.float().contiguous().clone())
        offset, ck = c.get("len", 0), {}
        seg = checkpoint_every or P
        conv = c.get("conv")
        for r0 in range(0, P, seg):
            r1 = min(P, r0 + seg)
            conv = ops.gdn_fill(pre[r0:r1], self.nk, self.nv, self.dk, self.dv, w["conv"], conv, w["a_log"],
                                w["dt_bias"], rec, self._gdn_workspace(r1 - r0, x.device))
            if checkpoint_every and r1 % checkpoint_every == 0:
                ck[offset + r1] = rec.clone()
        c["conv"], c["rec"] = conv, rec
        c["len"] = offset + P
        if st is not None:
            c["rec"] = c["rec"] + st.to(c["rec"])
        return ck

    def _fill_rows(self, w, x, ssq):
        """The in-projection rows [P, q | k | v | b | a] a GDN fill reads (code/kva/model.py:452-458). The state
        update reads k, v, b and a only, and the conv state the last 3 rows of q | k | v, so q is projected for
        those 3 rows alone and the other rows' q columns stay unwritten."""
        return self._fill_rows_batch([w], [x], [ssq])[0]

    def _fill_rows_batch(self, ws, xs, ssqs):
        """_fill_rows of several GDN layers over the same rows in one launch (ops.norm_linear_batch): per layer
        one entry of every row against the k | v | b | a rows and one of the last 3 rows against the q rows.
        Each value is the bits of the full projection of its row (the same kernel on the same row and weights)."""
        P = xs[0].shape[0]
        nq = self.nk * self.dk
        if nq % 256 or P <= 3 or any(x.stride(0) != xs[0].stride(0) for x in xs):
            return [ops.norm_linear(x, q, self.eps, w["w_in"]) for w, x, q in zip(ws, xs, ssqs)]
        pres = [torch.empty(P, w["w_in"].shape[0], dtype=torch.bfloat16, device=xs[0].device) for w in ws]
        ex, es, ew, eo = [], [], [], []
        for w, x, q, pre in zip(ws, xs, ssqs, pres):
            ex += [x, x[P - 3:]]
            es += [q, q[P - 3:]]
            ew += [w["w_in"][nq:], w["w_in"][:nq]]
            eo += [pre[:, nq:], pre[P - 3:, :nq]]
        ops.norm_linear_batch(ex, es, self.eps, ew, eo)
        return pres

    def fill_batch(self, ids, xs, cache, ssqs=None):
        """fill() of up to ops.GDN_BATCH_MAX GDN layers over the same rows at once: their in-projections in one launch
        (_fill_rows_batch), then one batched delta-rule fill (rf_gdn_fill_batch), so the layers' sequential chunk
        scans run side by side. Every layer's conv and recurrent state is bit-identical to fill() of it alone."""
        ids = list(ids)
        if not 1 <= len(ids) <= ops.GDN_BATCH_MAX or any(self.layer_types[i] != "gdn" for i in ids):
            raise ValueError(f"fill_batch: 1 .. {ops.GDN_BATCH_MAX} GDN layers, got {ids}")
        P = xs[0].shape[0]
        if any(x.shape[0] != P for x in xs):
            raise ValueError("fill_batch: every layer takes the same rows")
        if P == 0:
            return
        ssqs = [ops.row_ssq(x) if q is None else q for x, q in zip(xs, ssqs or [None] * len(ids))]
        pres = self._fill_rows_batch([self._layer(i, "gdn") for i in ids], xs, ssqs)
        jobs = []
        for i, x, ssq, pre in zip(ids, xs, ssqs, pres):
            w = self._layer(i, "gdn")
            c = cache[i]
            rec = c.get("rec")
            rec = (torch.zeros(self.nv, self.dk, self.dv, dtype=torch.float32, device=x.device) if rec is None
                   else rec.float().contiguous().clone())
            jobs.append((pre, w["conv"], c.get("conv"), w["a_log"], w["dt_bias"], rec))
        convs = ops.gdn_fill_batch(jobs, self.nk, self.nv, self.dk, self.dv,
                                   self._gdn_workspace(P, xs[0].device, len(ids)))
        for i, job, conv in zip(ids, jobs, convs):
            c = cache[i]
            c["conv"], c["rec"] = conv, job[5]
            c["len"] = c.get("len", 0) + P

    def _attn_workspace(self, nq, n, device):
        """The exact-row attention's key-split workspace, shared by every layer (stream-ordered reuse)."""
        need = ops.attend_rows_workspace_bytes(nq, self.n_heads, self.n_kv, self.head_dim, n)
        if need == 0:
            return None
        ws = getattr(self, "_attn_ws", None)
        if ws is None or ws.numel() < need or ws.device != device:
            self._attn_ws = ws = torch.empty(need, dtype=torch.uint8, device=device)
        return ws

    def gemm_workspace(self, M, N, K, device, role="consume", rows=False):
        """The split-K workspace of an M x N x K product (None when it runs unsplit): one buffer per role,
        shared by every GEMM of that role in stream order -- "consume" for the cache fill and the exact
        rows' and tail's layers, "produce" for the map apply that may run beside them on another stream.
        rows: size it for norm_kv_rows / norm_qkv_rows over M scattered rows (ops.rows_workspace_bytes)."""
        need = (ops.rows_workspace_bytes if rows else ops.gemm_workspace_bytes)(M, N, K)
        if need == 0:
            return None
        wss = self.__dict__.setdefault("_gemm_ws", {})
        ws = wss.get(role)
        if ws is None or ws.numel() < need or ws.device != device:
            wss[role] = ws = torch.empty(need, dtype=torch.uint8, device=device)
        return ws

    def _gdn_workspace(self, rows, device, layers=1):
        """The GDN kernels' per-chunk workspace, shared by every GDN layer (stream-ordered reuse), sized
        for min(rows, GDN_ROWS) rows per pass of one layer, or min(rows, GDN_BATCH_ROWS) of each of `layers`
        layers filled together. The kernels size their passes by the bytes they are given, so the view
        handed out is exactly that size, whatever larger buffer an earlier call left."""
        cap = GDN_ROWS if layers == 1 else GDN_BATCH_ROWS
        need = layers * ops.gdn_workspace_bytes(min(rows, cap), self.nk, self.nv, self.dk, self.dv)
        if self._gdn_ws is None or self._gdn_ws.numel() < need or self._gdn_ws.device != device:
            self._gdn_ws = None                         # the old buffer goes before the larger one is taken
            self._gdn_ws = torch.empty(need, dtype=torch.uint8, device=device)
        return self._gdn_ws[:need]

    def _pack_rows(self, i):
        """Layer i's weights for its full layer (exact rows, the exact tail), packed on first use, with the
        input norm gain folded into the projections (rf_fold_norm; the zero-centred 1 + g for Qwen3.5):
        attention -- the query projection (Qwen3.5: its query and output-gate halves apart), q_norm, o_proj;
        GDN -- the z projection, the gated output norm's weight, out_proj; every layer -- [gate; up] with
        the post-attention norm gain folded in (zero rows to a multiple of 256), down (zero columns to a
        multiple of 64)."""
        w = self._layer(i, self.layer_types[i])
        if "wo" in w:
            return w
        dev = lambda k: self._src[k].to(self.device, torch.bfloat16).contiguous()   # noqa: E731
        p = f"{self._pre}layers.{i}."
        kind = self.knorm_kind
        if w["kind"] == "attn":
            a = p + "self_attn."
            wq = dev(a + "q_proj.weight")
            if self.arch == "qwen3_5":                  # per head [q | gate] rows (code/kva/model.py:427-432)
                qg = wq.view(self.n_heads, 2, self.head_dim, wq.shape[1])
                w["wq"] = ops.fold_norm(qg[:, 0].reshape(-1, wq.shape[1]).contiguous(), w["ln1"], kind)
                w["wgate"] = ops.fold_norm(qg[:, 1].reshape(-1, wq.shape[1]).contiguous(), w["ln1"], kind)
            else:                                       # [wq; wkv] in one buffer: the exact rows' one product
                wqkv = torch.cat((ops.fold_norm(wq, w["ln1"], kind), w["wkv"]), 0)
                w["wqkv"], w["wq"], w["wkv"] = wqkv, wqkv[:wq.shape[0]], wqkv[wq.shape[0]:]
            if self.arch != "llama":
                w["q_norm"] = dev(a + "q_norm.weight")
            w["wo"] = dev(a + "o_proj.weight")
        else:
            a = p + "linear_attn."
            w["wz"] = ops.fold_norm(dev(a + "in_proj_z.weight"), w["ln1"], 1)
            w["gnorm"] = dev(a + "norm.weight")
            w["wo"] = dev(a + "out_proj.weight")
        gate, up = dev(p + "mlp.gate_proj.weight"), dev(p + "mlp.up_proj.weight")
        inter = gate.shape[0]
        gu = torch.cat((gate, up), 0)
        pad = (-gu.shape[0]) % 256
        if pad:
            gu = torch.cat((gu, gu.new_zeros(pad, gu.shape[1])), 0)
        w["wgu"] = ops.fold_norm(gu, dev(p + "post_attention_layernorm.weight"), kind)
        down = dev(p + "mlp.down_proj.weight")
        pad = (-inter) % 64
        if pad:
            down = torch.cat((down, down.new_zeros(down.shape[0], pad)), 1).contiguous()
        w["wd"], w["inter"] = down, inter
        return w

    def _gdn_forward_workspace(self, rows, device):
        need = ops.gdn_forward_workspace_bytes(rows, self.nk, self.nv, self.dk, self.dv)
        ws = getattr(self, "_gdn_fwd_ws", None)
        if ws is None or ws.numel() < need or ws.device != device:
            self._gdn_fwd_ws = ws = torch.empty(need, dtype=torch.uint8, device=device)
        return ws

    def _gdn_layer(self, i, h, ssq, cache, rows=None):
        """The exact GDN layer (code/kva/model.py:486-508; layer_rows :541-554): the in-projection, conv and
        delta rule with outputs over every row of h, continuing cache[i]'s conv and recurrent states, then
        for h (or its rows `rows`) the gated output norm with z, out_proj and its residual, and the MLP."""
        w = self._pack_rows(i)
        c = cache[i]
        T, H = h.shape
        pre = ops.norm_linear(h, ssq, self.eps, w["w_in"],
                              workspace=self.gemm_workspace(T, w["w_in"].shape[0], H, h.device))
        rec = c.get("rec")
        rec = (torch.zeros(self.nv, self.dk, self.dv, dtype=torch.float32, device=h.device) if rec is None
               else rec.float().contiguous().clone())
        out, conv = ops.gdn_forward(pre, self.nk, self.nv, self.dk, self.dv, w["conv"], c.get("conv"), w["a_log"],
                                    w["dt_bias"], rec, workspace=self._gdn_forward_workspace(T, h.device))
        c["conv"], c["rec"], c["len"] = conv, rec, c.get("len", 0) + T
        if rows is not None:
            out = ops.row_gather(out, rows)[0]
            h, ssq = ops.row_gather(h, rows)
        R = h.shape[0]
        z = ops.norm_linear(h, ssq, self.eps, w["wz"], workspace=self.gemm_workspace(R, w["wz"].shape[0], H, h.device))
        y = ops.gated_rms_norm(out, z, w["gnorm"], self.nv, self.dv, self.eps)
        return self._out_mlp(w, h, y)

    def _gate(self, w, x, ssq, o):
        """Qwen3.5's output gate: o * sigmoid(x_normed W_gate^T) in place (code/kva/model.py:444-445)."""
        if "wgate" in w:
            g = ops.norm_linear(x, ssq, self.eps, w["wgate"],
                                workspace=self.gemm_workspace(x.shape[0], w["wgate"].shape[0], x.shape[1], x.device))
            ops.sigmoid_mul(o, g, out=o)
        return o

    def layer_rows(self, i, x, pos, rows, cache, ssq=None, cs=None):
        """Fill cache[i] from the inputs x [P, H] of rows at positions pos (an empty cache, as fill()) and
        return the exact layer output of the rows x[rows] over that cache, [len(rows), H] bf16
        (code/kva/model.py:259-276): the rows' queries attend over the filled keys up to their own
        position, then o_proj, the residual, and the MLP with its residual. rows: sorted prefix rows.
        GDN layers (Qwen3.5): the delta rule runs with outputs over every row, the rest on the rows only."""
        c = cache[i]
        if c.get("n", 0) or c.get("len", 0):
            raise ValueError("layer_rows fills an empty cache (cache slot = position)")
        w = self._pack_rows(i)
        if ssq is None:
            ssq = ops.row_ssq(x)
        if self.layer_types[i] != "attn":
            return self._gdn_layer(i, x, ssq, cache, torch.as_tensor(rows, dtype=torch.int64).to(x.device))[0]
        if cs is None:
            cs = self.rope_table(pos)
        self.fill(i, x, pos, cache, ssq=ssq, cs=cs)
        rows = torch.as_tensor(rows, dtype=torch.int64).to(x.device)
        xr, sr = ops.row_gather(x, rows)
        H, R = xr.shape[1], xr.shape[0]
        q = ops.norm_q(xr, sr, self.eps, w["wq"], self.n_heads, self.head_dim, w.get("q_norm"), self.knorm_kind, cs,
                       rows, workspace=self.gemm_workspace(R, w["wq"].shape[0], H, x.device))
        qpos = pos.to(x.device, torch.int64)[rows]
        if self._causal_ok():
            o = ops.attend_causal(q, 0, c["kbuf"], c["vbuf"], c["n"], self.n_heads, self.scale, qpos=qpos,
                                  workspace=self._causal_workspace(R, c["n"], x.device))
        else:
            o = ops.attend_rows(q, qpos, c["kbuf"], c["vbuf"], c["n"], self.n_heads, self.scale,
                                workspace=self._attn_workspace(R, c["n"], x.device))
        return self._out_mlp(w, xr, self._gate(w, xr, sr, o))[0]

    def rows_over_fill(self, i, h, ssq, pos, rows, cache, cs, full=True, rows_max=None, qpos=None):
        """The exact rows' layer i over a cache already filled from every prefix row (fill() or
        fill_attn_batch() of the prefix rows' inputs, the rows' slots holding their fill values): the rows'
        own K / V, from their exact inputs h [R, H] (row sum-of-squares partials ssq), overwrite their slots
        (ops.norm_kv_rows), which leaves the cache layer_rows() builds by scattering the inputs in before the
        fill (code/kva/kva.py:392-454); then, if full, the rows' queries attend over the keys up to their own
        position, o_proj, the residual and the MLP (code/kva/model.py:259-276). Attention layers only: a GDN
        layer's fill carries the rows' inputs into every later state. rows: sorted prefix rows (int64 on the
        device), also their cache slots and table rows of cs (the RoPE table of pos); rows_max: a host bound on
        them; qpos: pos[rows] if already formed. Returns (output [R, H] bf16, its sum-of-squares partials), or
        None when not full."""
        if self.layer_types[i] != "attn":
            raise ValueError(f"rows_over_fill: layer {i} is {self.layer_types[i]}; attention layers only")
        c = cache[i]
        R, H = h.shape
        if not full:
            wl = self._layer(i)
            ops.norm_kv_rows(h, ssq, self.eps, wl["wkv"], self.n_kv, self.head_dim, wl.get("k_norm"),
                             self.knorm_kind, cs, rows, c["kbuf"], c["vbuf"], pos_max=rows_max,
                             workspace=self.gemm_workspace(R, wl["wkv"].shape[0], H, h.device, rows=True))
            return None
        w = self._pack_rows(i)
        if "wqkv" in w:                                 # queries and the rows' K / V from one product
            q = ops.norm_qkv_rows(h, ssq, self.eps, w["wqkv"], self.n_heads, self.n_kv, self.head_dim,
                                  w.get("q_norm"), w.get("k_norm"), self.knorm_kind, cs, rows, c["kbuf"], c["vbuf"],
                                  pos_max=rows_max,
                                  workspace=self.gemm_workspace(R, w["wqkv"].shape[0], H, h.device, rows=True))
        else:
            ops.norm_kv_rows(h, ssq, self.eps, w["wkv"], self.n_kv, self.head_dim, w.get("k_norm"), self.knorm_kind,
                             cs, rows, c["kbuf"], c["vbuf"], pos_max=rows_max,
                             workspace=self.gemm_workspace(R, w["wkv"].shape[0], H, h.device, rows=True))
            q = ops.norm_q(h, ssq, self.eps, w["wq"], self.n_heads, self.head_dim, w.get("q_norm"), self.knorm_kind,
                           cs, rows, workspace=self.gemm_workspace(R, w["wq"].shape[0], H, h.device))
        qpos = pos[rows] if qpos is None else qpos
        if self._causal_ok():
            o = ops.attend_causal(q, 0, c["kbuf"], c["vbuf"], c["n"], self.n_heads, self.scale, qpos=qpos,
                                  workspace=self._causal_workspace(R, c["n"], h.device))
        else:
            o = ops.attend_rows(q, qpos, c["kbuf"], c["vbuf"], c["n"], self.n_heads, self.scale,
                                workspace=self._attn_workspace(R, c["n"], h.device))
        return self._out_mlp(w, h, self._gate(w, h, ssq, o))

    def _out_mlp(self, w, h, o):
        """The rest of the layer after attention: h + o W_o^T, then the SwiGLU MLP with its residual
        (code/kva/model.py:112-118, :254-257), with the reference's bf16 roundings. Returns the layer
        output [rows, H] bf16 and its row sum-of-squares partials (the next norm's statistics)."""
        R, dev = h.shape[0], h.device
        gws = self.gemm_workspace
        h1, s1 = ops.map_apply_residual(o, w["wo"], h, workspace=gws(R, w["wo"].shape[0], w["wo"].shape[1], dev))
        inter = w["inter"]
        act = (torch.zeros if w["wd"].shape[1] != inter else torch.empty)(R, w["wd"].shape[1],
                                                                          dtype=torch.bfloat16, device=dev)
        wgu = w["wgu"]
        if wgu.shape[0] == 2 * inter and inter % 256 == 0:
            ops.norm_linear_swiglu(h1, s1, self.eps, wgu, out=act, workspace=gws(R, wgu.shape[0], wgu.shape[1], dev))
        else:                                           # [gate; up] padded to a multiple of 256 rows
            gu = ops.norm_linear(h1, s1, self.eps, wgu, workspace=gws(R, wgu.shape[0], wgu.shape[1], dev))
            ops.silu_mul(gu[:, :2 * inter], act[:, :inter])
        return ops.map_apply_residual(act, w["wd"], h1, workspace=gws(R, w["wd"].shape[0], w["wd"].shape[1], dev))

    def layer(self, i, h, pos, cache, ssq=None, cs=None):
        """Exact layer i for new rows h [T, H] bf16 at positions pos, appended after the cache's n rows
        (code/kva/model.py:247-257; the exact tail of finish(), code/kva/kva.py:457): K / V of the rows
        into slots n .. n + T - 1, the rows' queries attend causally over the keys up to their own slot
        (bottom-right aligned, as code/kva/ops.py:107-128), then o_proj, the residual and the MLP with its
        residual. ssq / cs: h's row sum-of-squares partials and the RoPE table of pos, if already built.
        Returns (layer output [T, H] bf16, its row sum-of-squares partials). GDN layers (Qwen3.5): the
        conv and delta rule continue the cache's states over the rows (code/kva/model.py:486-508)."""
        if ssq is None:
            ssq = ops.row_ssq(h)
        if self.layer_types[i] != "attn":
            return self._gdn_layer(i, h, ssq, cache)
        w = self._pack_rows(i)
        c = cache[i]
        T = h.shape[0]
        if cs is None:
            cs = self.rope_table(pos)
        slot = self.reserve(c, T, self.n_kv, self.head_dim, h.device)
        H = h.shape[1]
        ops.norm_kv_write(h, ssq, self.eps, w["wkv"], self.n_kv, self.head_dim, w.get("k_norm"), self.knorm_kind,
                          cs, c["kbuf"], c["vbuf"], slot,
                          workspace=self.gemm_workspace(T, w["wkv"].shape[0], H, h.device))
        self.commit(c, T)
        idx = torch.arange(T, device=h.device)
        q = ops.norm_q(h, ssq, self.eps, w["wq"], self.n_heads, self.head_dim, w.get("q_norm"), self.knorm_kind, cs,
                       idx, workspace=self.gemm_workspace(T, w["wq"].shape[0], H, h.device))
        if self._causal_ok():
            o = ops.attend_causal(q, slot, c["kbuf"], c["vbuf"], c["n"], self.n_heads, self.scale,
                                  workspace=self._causal_workspace(T, c["n"], h.device))
        else:
            o = ops.attend_rows(q, idx + slot, c["kbuf"], c["vbuf"], c["n"], self.n_heads, self.scale,
                                workspace=self._attn_workspace(T, c["n"], h.device))
        return self._out_mlp(w, h, self._gate(w, h, ssq, o))

    def embed(self, ids):
        """Embedding rows of token ids [T] (code/kva/model.py:108-109): a bit-exact row gather from the bf16
        table (kept on the device after the first call). Returns (h [T, H] bf16, its row sum-of-squares
        partials)."""
        if getattr(self, "_embed", None) is None:
            self._embed = self._src[self._pre + "embed_tokens.weight"].to(self.device, torch.bfloat16).contiguous()
        ids = torch.as_tensor(ids, dtype=torch.int64).to(self.device)
        if ids.dim() != 1:
            raise ValueError(f"ids: expected a 1-d tensor of token ids, got shape {tuple(ids.shape)}")
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self._embed.shape[0]):
            raise ValueError(f"ids: token ids must lie in [0, {self._embed.shape[0]})")
        return ops.row_gather(self._embed, ids)

    def forward_exact(self, ids, hook=None, cache=None, keep=None, stop=None):
        """Exact forward over all rows of one document (code/kva/model.py:167-181): hook(i, h) sees each
        layer's input h [T, H] bf16 and hook("final", h) the final-norm input; keep: row indices whose
        logits to return. stop: return after hook(stop, h), before layer `stop` runs (a capture that needs
        no later layer). Returns (logits of keep or None, cache)."""
        cache = self.new_cache() if cache is None else cache
        if any(c.get("n", 0) or c.get("len", 0) for c in cache):
            raise ValueError("forward_exact starts from an empty cache (cache slot = position)")
        h, ssq = self.embed(ids)
        pos = torch.arange(h.shape[0], device=self.device)
        cs = self.rope_table(pos)
        for i in range(self.n_layers):
            if hook is not None:
                hook(i, h)
            if i == stop:
                return None, cache
            h, ssq = self.layer(i, h, pos, cache, ssq=ssq, cs=cs)
        if hook is not None:
            hook("final", h)
        return (self.logits(h[torch.as_tensor(keep, device=self.device)]) if keep is not None else None), cache

    def _causal_workspace(self, nq, n, device):
        """rf_attend_causal's workspace (the key-range splits' partials), shared by every layer
        (stream-ordered reuse)."""
        need = ops.attend_causal_workspace_bytes(nq, self.n_heads, self.n_kv, self.head_dim, n)
        ws = getattr(self, "_causal_ws", None)
        if ws is None or ws.numel() < need or ws.device != device:
            self._causal_ws = ws = torch.empty(need, dtype=torch.uint8, device=device)
        return ws

    def _causal_ok(self):
        rep = self.n_heads // self.n_kv
        return (self.head_dim in (64, 128) and rep in ops.CAUSAL_GROUPS) or (self.head_dim == 256
                                                                           and rep in ops.CAUSAL_GROUPS_256)

    def logits(self, h, ssq=None):
        """F.linear(final_norm(h), lm_head).float() (code/kva/model.py:110-111): [rows, V] fp32 from bf16
        rows. The final norm's gain is folded into the packed lm_head (zero rows up to a multiple of 256)."""
        if getattr(self, "_lm", None) is None:
            src, pre = self._src, self._pre
            dev = lambda k: src[k].to(self.device, torch.bfloat16).contiguous()   # noqa: E731
            head = dev("lm_head.weight") if "lm_head.weight" in src else dev(pre + "embed_tokens.weight")
            V = head.shape[0]
            pad = (-V) % 256
            if pad:
                head = torch.cat((head, head.new_zeros(pad, head.shape[1])), 0)
            self._lm = (ops.fold_norm(head, dev(pre + "norm.weight"), self.knorm_kind), V)
        head, V = self._lm
        if ssq is None:
            ssq = ops.row_ssq(h)
        return ops.norm_linear(h, ssq, self.eps, head,
                               workspace=self.gemm_workspace(h.shape[0], head.shape[0], h.shape[1], h.device))[:, :V].float()

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
