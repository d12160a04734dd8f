"""A whole decode stack on one GPU: Transformer::forward
(crates/kestrel-engine/src/transformer.rs:278-302, 375-467) over libkmoe's
kernels, with every weight, the KV cache and the activations resident in HBM.

The model is given as kestrel's Transformer sees it: hyperparameters and GGUF
tensors by name (type, dims with the contiguous dimension first, bytes), so a
GGUF or KGUF reader hands its tensors over unchanged:

    hp:      arch, n_layer, n_embd, n_head, n_head_kv, head_dim, rope_dim,
             rope_freq_base, rms_eps, n_ctx, n_batch; MoE models add
             n_expert, n_expert_used, norm_topk, weights_scale
    tensors: "token_embd.weight", "output_norm.weight", optional
             "output.weight" (tied to the embedding when absent),
             "rope_freqs.weight"; per layer "blk.{l}.attn_norm.weight",
             attn_{q,k,v,output}.weight, optional attn_{q,k,v}.bias and
             attn_{q,k}_norm.weight, ffn_norm.weight, then either dense
             ffn_{gate,up,down}.weight or routed ffn_gate_inp.weight +
             ffn_{gate,up,down}_exps.weight (+ the *_shexp shared expert).

Layers with routed experts go through kmoe_moe_ffn and its HBM expert tier;
the rest through the decoder ops of include/kmoe.h. A single-token decode
step reads its position from a device counter, so it is captured once as a
HIP graph and replayed for every later token (greedy decoding keeps the
sampled token on the device too).
"""
from __future__ import annotations

import numpy as np

from .kmoe import BLOCK, F32, Context, bytes_for


def _nbytes(t: int, dims) -> int:
    rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
    return bytes_for(t, dims[0]) * rows


class Decoder:
    """Transformer::forward on the GPU (see the module docstring)."""

    def __init__(self, ctx: Context, hp: dict, tensors: dict, layer_base: int = 1000):
        torch = ctx.torch
        self.ctx, self.hp, self.torch = ctx, hp, torch
        self.d, self.nh, self.nkv, self.hd = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        self.rd, self.eps = hp["rope_dim"], float(hp["rms_eps"])
        self.neox = hp["arch"] != "llama"
        self.n_ctx, self.n_batch = hp["n_ctx"], max(1, hp.get("n_batch", 512))
        self.n_layer = hp["n_layer"]
        if self.nh % self.nkv:
            raise ValueError("n_head must be a multiple of n_head_kv")
        dev = f"cuda:{ctx.device}"
        self.dev = dev
        self._raw = {}

        def raw(name):
            ty, dims, b = tensors[name]
            b = np.ascontiguousarray(b, dtype=np.uint8).reshape(-1)
            if b.size < _nbytes(ty, dims):
                raise ValueError(f"{name}: {b.size} bytes < {_nbytes(ty, dims)}")
            t = torch.from_numpy(b).to(dev)
            self._raw[name] = (ty, list(dims), t)
            return self._raw[name]

        def vec(name):
            """An F32/F16/quantized vector as f32 on the device (dequantized by the device row kernel)."""
            ty, dims, t = raw(name)
            n = int(np.prod(dims))
            if ty == F32:
                return t[:4 * n].view(torch.float32).clone()
            return ctx.get_rows(ty, t, 1, n, [0]).reshape(n)

        self.embed = raw("token_embd.weight")
        self.n_vocab = self.embed[1][1]
        self.out_norm = vec("output_norm.weight")
        self.head = raw("output.weight") if "output.weight" in tensors else self.embed
        inv = None
        freqs = vec("rope_freqs.weight") if "rope_freqs.weight" in tensors else None
        base = np.float32(hp["rope_freq_base"])
        e = (-(2.0 * np.arange(self.rd // 2, dtype=np.float32)) / np.float32(self.rd)).astype(np.float32)
        inv = torch.from_numpy(np.power(base, e, dtype=np.float32)).to(dev)
        if freqs is not None:
            inv = inv / freqs
        self.inv_freq = inv.contiguous()

        kvw = self.nkv * self.hd
        self.layers = []
        for l in range(self.n_layer):
            p = f"blk.{l}."
            L = {"attn_norm": vec(p + "attn_norm.weight"), "ffn_norm": vec(p + "ffn_norm.weight"),
                 "wo": raw(p + "attn_output.weight")}
            wq, wk, wv = (tensors[p + f"attn_{n}.weight"] for n in "qkv")
            if wq[0] == wk[0] == wv[0]:  # one matmul over the concatenated rows (rows are independent)
                cat = np.concatenate([np.ascontiguousarray(w[2], dtype=np.uint8).reshape(-1)[:_nbytes(w[0], w[1])]
                                      for w in (wq, wk, wv)])
                L["wqkv"] = (wq[0], [wq[1][0], self.nh * self.hd + 2 * kvw], torch.from_numpy(cat).to(dev))
            else:
                L["wq"], L["wk"], L["wv"] = (raw(p + f"attn_{n}.weight") for n in "qkv")
            for n in "qkv":
                if p + f"attn_{n}.bias" in tensors:
                    L["b" + n] = vec(p + f"attn_{n}.bias")
            for n in "qk":
                if p + f"attn_{n}_norm.weight" in tensors:
                    L[n + "_norm"] = vec(p + f"attn_{n}_norm.weight")
            if p + "ffn_gate_exps.weight" in tensors:
                L["moe"] = self._moe_layer(l, layer_base + l, tensors)
            else:
                wg, wu = tensors[p + "ffn_gate.weight"], tensors[p + "ffn_up.weight"]
                if wg[0] == wu[0] and list(wg[1]) == list(wu[1]):  # gate | up rows in one matmul
                    cat = np.concatenate([np.ascontiguousarray(w[2], dtype=np.uint8).reshape(-1)[:_nbytes(w[0], w[1])]
                                          for w in (wg, wu)])
                    L["wgu"] = (wg[0], [wg[1][0], 2 * wg[1][1]], torch.from_numpy(cat).to(dev))
                else:
                    L["gate"], L["up"] = raw(p + "ffn_gate.weight"), raw(p + "ffn_up.weight")
                L["down"] = raw(p + "ffn_down.weight")
            L["kc"] = torch.zeros((self.n_ctx, kvw), dtype=torch.int16, device=dev)
            L["vc"] = torch.zeros((self.n_ctx, kvw), dtype=torch.int16, device=dev)
            self.layers.append(L)
        self.cached = 0
        self.pos_dev = torch.zeros(1, dtype=torch.int32, device=dev)
        self.token_dev = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graph = None
        self._graph_gen = None  # the context's workspace generation the graph was captured at
        self._graph_bufs = None

    def _moe_layer(self, l: int, lid: int, tensors: dict) -> int:
        ctx, hp, p = self.ctx, self.hp, f"blk.{l}."
        E = hp["n_expert"]
        g, u, dn = (tensors[p + f"ffn_{n}_exps.weight"] for n in ("gate", "up", "down"))
        ff = g[1][1]
        ctx.layer_create(lid, E, hp["n_expert_used"], self.d, ff, g[0], u[0], dn[0], hp.get("norm_topk", True),
                         hp.get("weights_scale", 0.0))
        rty, rdims, rb = tensors[p + "ffn_gate_inp.weight"]
        if rty != F32:
            raise ValueError("the router (ffn_gate_inp) must be F32, as kestrel's moe_ffn reads it")
        ctx.router_upload(lid, np.ascontiguousarray(rb, dtype=np.uint8).view(np.float32)[:E * self.d].reshape(E, self.d))
        for k, (ty, dims, b) in enumerate((g, u, dn)):
            b = np.ascontiguousarray(b, dtype=np.uint8).reshape(-1)
            sl = _nbytes(ty, dims) // E
            for e in range(E):
                ctx.expert_upload(lid, e, k, b[e * sl:(e + 1) * sl])
        if p + "ffn_gate_shexp.weight" in tensors:
            ts = [tensors[p + f"ffn_{n}_shexp.weight"] for n in ("gate", "up", "down")]
            gi = None
            if p + "ffn_gate_inp_shexp.weight" in tensors:
                gty, gdims, gb = tensors[p + "ffn_gate_inp_shexp.weight"]
                if gty != F32:
                    raise ValueError("ffn_gate_inp_shexp must be F32")
                gi = np.ascontiguousarray(gb, dtype=np.uint8).view(np.float32)[:self.d]
            ctx.shared_expert(lid, ts[0][1][1], [t[0] for t in ts], *[t[2] for t in ts], gate_inp=gi)
        return lid

    # ------------------------------------------------------------------ steps
    def _mm(self, w, x):
        ty, dims, t = w
        return self.ctx.matmul(ty, t, int(np.prod(dims[1:])), dims[0], x)

    def _layer(self, L, x, f_prev, S: int, pos0: int, pos_dev, spare=None):
        """One decoder layer on the residual stream x [S, d]. f_prev, the
        previous layer's FFN output, joins x in the first norm's fused add.
        Returns the layer's own FFN output and the buffer that now holds the
        residual stream: x (updated in place), or spare, a second buffer that
        one-token layers write x + f_prev into (x is then left as it was)."""
        ctx, nh, nkv, hd = self.ctx, self.nh, self.nkv, self.hd
        kvw, nq = nkv * hd, nh * hd
        plain = not any(n in L for n in ("bq", "bk", "bv", "q_norm", "k_norm"))
        if "wqkv" in L and S == 1 and plain:
            # one token: the projection kernel takes the residual add and the
            # norm (into the other buffer), applies RoPE and fills the caches
            ty, dims, t = L["wqkv"]
            xr = x if spare is None else spare
            qr = ctx.norm_matmul_rope_kv(x, L["attn_norm"], self.eps, ty, t, dims[0], nh, nkv, hd, self.rd, pos0,
                                         self.inv_freq, self.neox, self.n_ctx, L["kc"], L["vc"], y=f_prev,
                                         pos_dev=pos_dev, x_out=spare)
            return self._attn_ffn(L, xr, qr, S, pos0, pos_dev), xr
        if "wqkv" in L:
            ty, dims, t = L["wqkv"]
            qkv = ctx.norm_matmul(x, L["attn_norm"], self.eps, ty, t, dims[1], dims[0], y=f_prev)
            q, k, v = qkv[:, :nq], qkv[:, nq:nq + kvw], qkv[:, nq + kvw:]
            if S > 1:
                q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        else:
            h = ctx.rmsnorm(x, L["attn_norm"], self.eps, y=f_prev)
            q, k, v = self._mm(L["wq"], h), self._mm(L["wk"], h), self._mm(L["wv"], h)
        for n, y in (("q", q), ("k", k), ("v", v)):
            if "b" + n in L:
                ctx.add_rows(y, L["b" + n])
        if "q_norm" in L:
            ctx.rmsnorm(q, L["q_norm"], self.eps, out=q)
        if "k_norm" in L:
            ctx.rmsnorm(k, L["k_norm"], self.eps, out=k)
        qr = ctx.rope_kv_store(q, k, v, nh, nkv, hd, self.rd, pos0, self.inv_freq, self.neox, self.n_ctx, L["kc"],
                               L["vc"], pos_dev)
        return self._attn_ffn(L, x, qr, S, pos0, pos_dev), x

    def _attn_ffn(self, L, x, qr, S, pos0, pos_dev):
        """Attention from the rotated q and the caches, its projection, then the FFN."""
        ctx, nh, nkv, hd = self.ctx, self.nh, self.nkv, self.hd
        ty, dims, t = L["wo"]
        o = ctx.attention_matmul(qr, L["kc"], L["vc"], nh, nkv, hd, pos0, self.n_ctx, ty, t,
                                 int(np.prod(dims[1:])), pos_dev)
        if "moe" in L:
            # x += o, the norm of x, then the routed experts (one token: the
            # router kernel takes the norm)
            return ctx.norm_moe_ffn(L["moe"], x, L["ffn_norm"], self.eps, y=o)
        if "wgu" in L:
            ty, dims, t = L["wgu"]
            ff = dims[1] // 2
            gu = ctx.norm_matmul(x, L["ffn_norm"], self.eps, ty, t, dims[1], dims[0], y=o)
            g, u = gu[:, :ff], gu[:, ff:]
            if S > 1:
                g, u = g.contiguous(), u.contiguous()
        else:
            h = ctx.rmsnorm(x, L["ffn_norm"], self.eps, y=o)
            g, u = self._mm(L["gate"], h), self._mm(L["up"], h)
        return self._mm(L["down"], ctx.swiglu(g, u))

    def _stack(self, x, S: int, pos0: int, pos_dev):
        """All layers and the head; returns the logits of the last row."""
        f = None
        spare = self.torch.empty_like(x) if S == 1 else None  # the residual stream's second buffer
        for L in self.layers:
            f, xr = self._layer(L, x, f, S, pos0, pos_dev, spare)
            if xr is not x:
                x, spare = xr, x
        ty, dims, t = self.head
        return self.ctx.norm_matmul(x[S - 1:S], self.out_norm, self.eps, ty, t, dims[1], dims[0],
                                    y=f[S - 1:S]).reshape(-1)

    def forward(self, tokens):
        """Transformer::forward: feed host token ids; returns the last row's
        logits (f32 [n_vocab], on the device)."""
        tokens = [int(t) for t in tokens]
        if not tokens:
            raise ValueError("forward() needs at least one token")
        if self.cached + len(tokens) > self.n_ctx:
            raise ValueError(f"context full: need {self.cached + len(tokens)}, n_ctx {self.n_ctx}")
        logits = None
        for i in range(0, len(tokens), self.n_batch):
            chunk = tokens[i:i + self.n_batch]
            ty, dims, t = self.embed
            x = self.ctx.get_rows(ty, t, dims[1], dims[0], chunk)
            logits = self._stack(x, len(chunk), self.cached, None)
            self.cached += len(chunk)
        return logits

    # --------------------------------------------------------- greedy decode
    def _decode_body(self):
        ty, dims, t = self.embed
        x = self.ctx.get_rows(ty, t, dims[1], dims[0], self.token_dev, out=self._graph_bufs["x"])
        logits = self._stack(x, 1, 0, self.pos_dev)
        self._graph_bufs["logits"] = logits
        self.ctx.argmax(logits, out=self.token_dev, pos_dev=self.pos_dev, advance=1)

    def decode_greedy(self, first_token: int, n: int, use_graph: bool = True):
        """Greedy decoding (sampler.rs:58-59): feed first_token, then each
        argmax, n steps; returns the n sampled ids. One step = one token
        through every layer, the head and argmax, all on the device; with
        use_graph the step is captured once and replayed."""
        torch = self.torch
        if self.cached + n > self.n_ctx:
            raise ValueError("context full")
        self.pos_dev.fill_(self.cached)
        self.token_dev.fill_(int(first_token))
        if self._graph_bufs is None:
            self._graph_bufs = {"x": torch.empty((1, self.d), dtype=torch.float32, device=self.dev)}
        out = torch.empty(n, dtype=torch.int32, device=self.dev)
        if not use_graph:
            for i in range(n):
                self._decode_body()
                out[i:i + 1].copy_(self.token_dev)
            self.cached += n
            return out
        if self.graph is not None and self.ctx.workspace_generation() != self._graph_gen:
            # a workspace the graph points into was reallocated since the capture
            # (a longer prompt chunk, another caller of the context): capture again
            self.graph = None
        if self.graph is None:
            # warm-up call at the same shapes grows every workspace first
            pos, tok = self.pos_dev.clone(), self.token_dev.clone()
            self._decode_body()
            self.pos_dev.copy_(pos)
            self.token_dev.copy_(tok)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            try:
                with torch.cuda.graph(g):
                    self.ctx.set_stream(torch.cuda.current_stream())  # the capturing stream
                    self._decode_body()
            finally:
                self.ctx.set_stream(torch.cuda.current_stream())
            self.graph = g
            self._graph_gen = self.ctx.workspace_generation()
            torch.cuda.synchronize()
        for i in range(n):
            self.graph.replay()
            out[i:i + 1].copy_(self.token_dev)
        self.cached += n
        return out

    def close(self):
        for L in self.layers:
            if "moe" in L:
                self.ctx.layer_destroy(L["moe"])
        self.layers = []
        self.graph = None


__all__ = ["Decoder", "BLOCK"]
