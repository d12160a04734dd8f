"""Shared input builders for the parity tests (seeded; identical bytes go to
the oracle and to the GPU)."""
from __future__ import annotations

import numpy as np

F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def row_bytes(t: int, cols: int) -> int:
    bs, ts = BLOCK[t]
    return cols // bs * ts


def f16_bytes(v: float) -> np.ndarray:
    return np.array([v], np.float16).view(np.uint8)


def random_blocks(t: int, rows: int, cols: int, seed: int, d: float | None = None,
                  dmin: float | None = None) -> np.ndarray:
    """Well-formed blocks of random bytes with f16 scales overwritten, the way
    the reference's kernel tests build them (avx2.rs:198-208, qdot.rs:275-299).
    Defaults give weights of std ~0.02 (Q4_K: dmin = 7.5 d centres them; Q6_K
    has its f16 d at byte 208)."""
    rng = np.random.default_rng(seed)
    bs, ts = BLOCK[t]
    nb = rows * cols // bs
    raw = rng.integers(0, 256, size=(nb, ts), dtype=np.uint8)
    if t == Q4_K:
        d = 1.4e-4 if d is None else d
        dmin = 7.5 * d if dmin is None else dmin
        raw[:, 0:2] = f16_bytes(d)
        raw[:, 2:4] = f16_bytes(dmin)
    elif t == Q6_K:  # q - 32 uniform (std ~18.5), sc uniform int8 (rms ~74): d*74*18.5 ~ 0.02
        d = 1.5e-5 if d is None else d
        raw[:, 208:210] = f16_bytes(d)
    else:
        d = 0.02 / 74.0 if d is None else d
        raw[:, 0:2] = f16_bytes(d)
    return raw.reshape(-1)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


class LayerSpec:
    """One MoE layer's host-side tensors (GGUF bytes per expert, f32 router)."""

    def __init__(self, n_expert, k, d, ff, wtype, seed=0, quantized=True, norm_topk=True, weights_scale=0.0,
                 down_type=None, zipf=None):
        from oracle import pyoracle as orc

        self.n_expert, self.k, self.d, self.ff = n_expert, k, d, ff
        self.gate_type = self.up_type = wtype
        self.down_type = wtype if down_type is None else down_type
        self.norm_topk, self.weights_scale = norm_topk, weights_scale
        s = seed * 7919
        self.router = orc.normal(s + 1, n_expert * d, 0.0, 0.02).reshape(n_expert, d)
        if zipf is not None:
            # Zipf(s) load imbalance through the unchanged routing function: a
            # rank-1 term along the all-ones direction of the router rows; with
            # activations offset by +1 it adds log(zipf weight) to the logits.
            rng = np.random.default_rng(seed + 17)
            rank = rng.permutation(n_expert) + 1
            bias = -zipf * np.log(rank.astype(np.float64))
            self.router = (self.router + (bias / d)[:, None]).astype(np.float32)

        def mk(sd, t, r, c):
            if quantized:
                return orc.quantize(t, orc.normal(sd, r * c, 0.0, 0.02).reshape(r, c))
            return random_blocks(t, r, c, sd)

        self.gate = [mk(s + 100 + e, self.gate_type, ff, d) for e in range(n_expert)]
        self.up = [mk(s + 200 + e, self.up_type, ff, d) for e in range(n_expert)]
        self.down = [mk(s + 300 + e, self.down_type, d, ff) for e in range(n_expert)]

    def oracle_layer(self):
        from oracle import pyoracle as orc

        return orc.Layer(self.n_expert, self.k, self.d, self.ff, self.gate_type, self.up_type, self.down_type,
                         self.router, self.gate, self.up, self.down, self.norm_topk, self.weights_scale)

    def upload(self, ctx, layer: int = 0):
        ctx.layer_create(layer, self.n_expert, self.k, self.d, self.ff, self.gate_type, self.up_type,
                         self.down_type, self.norm_topk, self.weights_scale)
        ctx.router_upload(layer, self.router)
        for e in range(self.n_expert):
            ctx.expert_upload(layer, e, 0, self.gate[e])
            ctx.expert_upload(layer, e, 1, self.up[e])
            ctx.expert_upload(layer, e, 2, self.down[e])


def _align(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def expert_images(spec: "LayerSpec", seed: int = 0, align: int = 32, page: int = 4096):
    """The layer's routed experts as the two file layouts hold them, each an
    image of host bytes with junk in every gap, and (part offsets, strides):

    - plain GGUF: three stacked tensors ffn_{gate,up,down}_exps, each at an
      `align`-aligned offset, expert e's slice at offset + e * slice_bytes
      (TensorInfo::slice_offset, kestrel-gguf/src/lib.rs:187-189);
    - prepared KGUF: expert e is [gate_e | up_e | down_e] with each part
      `align`-aligned inside the block and the block padded to a page; the
      three tensors share that stride (kestrel-model/src/prepare.rs:118-131).
    """
    rng = np.random.default_rng(seed + 99)
    parts = (spec.gate, spec.up, spec.down)
    s = [len(p[0]) for p in parts]
    E = spec.n_expert
    # plain: a page of other tensors first, then the three stacked tensors
    off = [page + 64]
    for k in (1, 2):
        off.append(_align(off[-1] + E * s[k - 1], align))
    plain = rng.integers(0, 256, off[2] + E * s[2] + 100, dtype=np.uint8)
    for k in range(3):
        for e in range(E):
            plain[off[k] + e * s[k]:off[k] + (e + 1) * s[k]] = parts[k][e]
    plain_layout = (off, s)
    # prepared: page-aligned group start, parts aligned inside a page-padded block
    o = [0, _align(s[0], align)]
    o.append(_align(o[1] + s[1], align))
    stride = _align(o[2] + s[2], page)
    start = 2 * page
    kg = rng.integers(0, 256, start + E * stride, dtype=np.uint8)
    for e in range(E):
        for k in range(3):
            b = start + e * stride + o[k]
            kg[b:b + s[k]] = parts[k][e]
    kg_layout = ([start + x for x in o], [stride] * 3)
    return (plain, plain_layout), (kg, kg_layout)


def decoder_model(arch: str = "llama", n_layer: int = 2, d: int = 256, nh: int = 4, nkv: int = 2, hd: int = 64,
                  ff: int = 512, vocab: int = 1000, n_ctx: int = 256, n_batch: int = 512, moe: dict | None = None,
                  wtype: int = Q4_K, embed_type: int = Q8_0, head_type: int | None = Q6_K, bias: bool = False,
                  qk_norm: bool = False, shared_ff: int = 0, seed: int = 0, rope_dim: int | None = None):
    """A small decoder as kestrel's Transformer reads it: (hp, tensors) with
    GGUF names, tensors = name -> (ggml type, dims with the contiguous
    dimension first, bytes). Weights are the oracle's quantization of
    seeded normals; norms are 1 + N(0, 0.1). head_type None ties the output
    to the embedding. moe = dict(n_expert, n_expert_used, norm_topk,
    weights_scale, types=(gate, up, down))."""
    from oracle import pyoracle as orc

    s = [seed * 1000 + 1]

    def normal(n, std=1.0, mean=0.0):
        s[0] += 1
        return orc.normal(s[0], n, mean, std)

    def mat(t, rows, cols, std):
        return (t, [cols, rows], orc.quantize(t, normal(rows * cols, std).reshape(rows, cols)))

    def f32(v, dims):
        v = np.ascontiguousarray(v, dtype=np.float32)
        return (F32, list(dims), v.view(np.uint8).reshape(-1))

    hp = dict(arch=arch, n_layer=n_layer, n_embd=d, n_head=nh, n_head_kv=nkv, head_dim=hd,
              rope_dim=rope_dim or hd, rope_freq_base=10000.0, rms_eps=1e-5, n_ctx=n_ctx, n_batch=n_batch)
    T = {"token_embd.weight": mat(embed_type, vocab, d, 1.0),
         "output_norm.weight": f32(1.0 + normal(d, 0.1), [d])}
    if head_type is not None:
        T["output.weight"] = mat(head_type, vocab, d, 0.05)
    if moe:
        hp.update(n_expert=moe["n_expert"], n_expert_used=moe["n_expert_used"],
                  norm_topk=moe.get("norm_topk", True), weights_scale=moe.get("weights_scale", 0.0))
    for l in range(n_layer):
        p = f"blk.{l}."
        T[p + "attn_norm.weight"] = f32(1.0 + normal(d, 0.1), [d])
        T[p + "ffn_norm.weight"] = f32(1.0 + normal(d, 0.1), [d])
        T[p + "attn_q.weight"] = mat(wtype, nh * hd, d, 0.08)
        T[p + "attn_k.weight"] = mat(wtype, nkv * hd, d, 0.08)
        T[p + "attn_v.weight"] = mat(wtype, nkv * hd, d, 0.05)
        T[p + "attn_output.weight"] = mat(wtype, d, nh * hd, 0.05)
        if bias:
            for n, w in (("q", nh * hd), ("k", nkv * hd), ("v", nkv * hd)):
                T[p + f"attn_{n}.bias"] = f32(normal(w, 0.1), [w])
        if qk_norm:
            T[p + "attn_q_norm.weight"] = f32(1.0 + normal(hd, 0.1), [hd])
            T[p + "attn_k_norm.weight"] = f32(1.0 + normal(hd, 0.1), [hd])
        if moe:
            E = moe["n_expert"]
            tg, tu, tdn = moe.get("types", (wtype, wtype, wtype))
            T[p + "ffn_gate_inp.weight"] = f32(normal(E * d, 0.05), [d, E])
            for n, t, rows, cols in (("gate", tg, ff, d), ("up", tu, ff, d), ("down", tdn, d, ff)):
                b = np.concatenate([orc.quantize(t, normal(rows * cols, 0.03).reshape(rows, cols))
                                    for _ in range(E)])
                T[p + f"ffn_{n}_exps.weight"] = (t, [cols, rows, E], b)
            if shared_ff:
                T[p + "ffn_gate_shexp.weight"] = mat(wtype, shared_ff, d, 0.03)
                T[p + "ffn_up_shexp.weight"] = mat(wtype, shared_ff, d, 0.03)
                T[p + "ffn_down_shexp.weight"] = mat(Q8_0, d, shared_ff, 0.03)
                T[p + "ffn_gate_inp_shexp.weight"] = f32(normal(d, 0.05), [d])
        else:
            T[p + "ffn_gate.weight"] = mat(wtype, ff, d, 0.03)
            T[p + "ffn_up.weight"] = mat(wtype, ff, d, 0.03)
            T[p + "ffn_down.weight"] = mat(wtype, d, ff, 0.03)
    return hp, T


def midpoint_rows(rows: int, cols: int, block: int, seed: int):
    """Activation rows whose int8 quantization (Q8Row per 32, Q8KRow per 256;
    qdot.rs:30-49, :347-367) lands on exact rounding midpoints.

    Each block's largest magnitude is 127 * 2^e, so scale = amax / 127 = 2^e
    and inv = 2^-e are exact, and every other element is +-(m + 0.5) * 2^e
    (m in 0..126, even and odd) or an integer multiple of 2^e, so x * inv is
    exact too. Returns (x f32 [rows, cols], t = x / 2^e as float64): the
    expected int8 value is sign(t) * floor(|t| + 0.5) (f32::round, half away
    from zero), which differs from round-half-even wherever m is even."""
    rng = np.random.default_rng(seed)
    nb = cols // block
    e = rng.integers(-7, 3, size=(rows, nb))
    m = rng.integers(0, 127, size=(rows, nb, block)).astype(np.float64)
    half = rng.random((rows, nb, block)) < 0.85
    t = np.where(half, m + 0.5, m) * np.where(rng.random((rows, nb, block)) < 0.5, -1.0, 1.0)
    pos = rng.integers(0, block, size=(rows, nb))
    r_i, b_i = np.meshgrid(np.arange(rows), np.arange(nb), indexing="ij")
    t[r_i, b_i, pos] = np.where(rng.random((rows, nb)) < 0.5, -127.0, 127.0)
    x = (t * np.ldexp(1.0, e)[:, :, None]).astype(np.float32)
    assert np.array_equal(x.astype(np.float64), t * np.ldexp(1.0, e)[:, :, None])  # exact in f32
    return x.reshape(rows, cols), t.reshape(rows, cols)


def round_half_away(t: np.ndarray) -> np.ndarray:
    """Rust f32::round then clamp(-127, 127) as i8, on exact float64 values."""
    return np.clip(np.sign(t) * np.floor(np.abs(t) + 0.5), -127, 127).astype(np.int8)


# ---------------------------------------------------------------- decode stacks

def synthetic_blocks(t: int, n_blocks: int, scale: float, rng):
    """Random well-formed blocks with dequantized std ~scale, built the way
    kestrel's synthetic models are (tools/make_synthetic.py:38-58): Q4_K with
    every 6-bit scale and min at 32 and dmin = 7.5 d (zero-mean weights), Q6_K
    with int8 scales 16..47, Q8_0 uniform int8 under one scale."""
    f16 = lambda v: np.frombuffer(np.float16(v).tobytes(), np.uint8)
    if t == Q8_0:  # uniform int8 weights (std ~74) under one f16 scale
        raw = rng.integers(0, 256, size=(n_blocks, 34), dtype=np.uint8)
        raw[:, 0:2] = f16(scale / 74.0)
        return raw.reshape(-1)
    if t == Q4_K:
        raw = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
        d = scale / (32 * 4.61)
        raw[:, 0:2] = f16(d)
        raw[:, 2:4] = f16(7.5 * d)
        raw[:, 4:16] = np.array([160] * 8 + [0] * 4, np.uint8)
    else:
        raw = rng.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
        raw[:, 192:208] = (raw[:, 192:208] % 32 + 16).astype(np.uint8)
        raw[:, 208:210] = f16(scale / 600.0)
    return raw.reshape(-1)


MOE6B = dict(name="synthetic moe-6b (llama arch)", arch="llama", layers=24, embd=2048, ff=1536, heads=16,
             kv_heads=4, vocab=32000, experts=32, experts_used=4, norm_topk=False, weights_scale=0.0,
             down_type=Q4_K, shared_ff=0, dense_layers=0, dense_ff=0)
# DeepSeek-V2-Lite's shape as kestrel can hold it: qwen2moe (the reference's
# native MoE architecture with shared experts; deepseek2 itself is
# LlamaCppOnly, kestrel-model/src/adapters.rs:32) with plain multi-head
# attention in place of MLA, 27 layers of which the first is dense (FFN
# 10944, first_k_dense_replace = 1), 64 routed experts of FFN 1408, top-6
# with unrenormalised softmax weights, 2 shared experts as one ungated FFN of
# 2816; Q4_K_M-style types: Q4_K, Q8_0 where a row is not a multiple of 256
# (routed down, dense down), Q6_K shared down and head.
DSV2LITE = dict(name="DeepSeek-V2-Lite-shaped (qwen2moe arch, MHA)", arch="qwen2moe", layers=27, embd=2048,
                ff=1408, heads=16, kv_heads=16, vocab=102400, experts=64, experts_used=6, norm_topk=False,
                weights_scale=1.0, down_type=Q8_0, shared_ff=2816, dense_layers=1, dense_ff=10944)
STACKS = {"moe6b": MOE6B, "dsv2lite": DSV2LITE}


def tensor_bytes(t: int, rows: int, cols: int) -> int:
    return rows * row_bytes(t, cols)


def stack_model(c: dict, rng, n_ctx: int, n_layer: int | None = None, share: bool = True):
    """(hp, tensors) of a synthetic decode stack of config c (MOE6B or
    DSV2LITE) as Transformer::forward reads it (GGUF names, dims with the
    contiguous dimension first): Q4_K embedding, Q6_K head, Q4_K attention,
    routed experts Q4_K / Q4_K / c["down_type"], the dense layers' FFN
    Q4_K / Q4_K / Q8_0, the shared FFN Q4_K / Q4_K / Q6_K; random well-formed
    blocks, unit norm weights, routers N(0, 16/d) per layer. n_layer cuts the
    depth (the dense layers stay first). share: attention, expert and dense
    bytes are one host array for all layers (each layer still gets its own
    copy in HBM); otherwise every layer draws its own."""
    L = c["layers"] if n_layer is None else n_layer
    d, ff, H, KV, V, NE, NU = (c[k] for k in ("embd", "ff", "heads", "kv_heads", "vocab", "experts",
                                              "experts_used"))
    dt, FS, ND, FD = c["down_type"], c["shared_ff"], min(c["dense_layers"], L), c["dense_ff"]
    hd = d // H
    blk = {Q8_0: 32, Q4_K: 256, Q6_K: 256}
    mat = lambda t, rows, cols, sc: (t, [cols, rows], synthetic_blocks(t, rows * cols // blk[t], sc, rng))
    f32 = lambda v, dims: (F32, list(dims), np.ascontiguousarray(v, np.float32).view(np.uint8).reshape(-1))
    hp = dict(arch=c["arch"], n_layer=L, n_embd=d, n_head=H, n_head_kv=KV, head_dim=hd, rope_dim=hd,
              rope_freq_base=10000.0, rms_eps=1e-5, n_ctx=n_ctx, n_batch=512, n_expert=NE,
              n_expert_used=NU, norm_topk=c["norm_topk"], weights_scale=c["weights_scale"])
    T = {"token_embd.weight": mat(Q4_K, V, d, 1.0), "output_norm.weight": f32(np.ones(d), [d]),
         "output.weight": mat(Q6_K, V, d, 1.0 / np.sqrt(d))}
    s_d = 1 / np.sqrt(d)

    def attn():
        return {"attn_q.weight": mat(Q4_K, H * hd, d, s_d), "attn_k.weight": mat(Q4_K, KV * hd, d, s_d),
                "attn_v.weight": mat(Q4_K, KV * hd, d, s_d), "attn_output.weight": mat(Q4_K, d, H * hd, s_d)}

    def experts():
        return ((Q4_K, [d, ff, NE], synthetic_blocks(Q4_K, NE * ff * d // 256, s_d, rng)),
                (Q4_K, [d, ff, NE], synthetic_blocks(Q4_K, NE * ff * d // 256, s_d, rng)),
                (dt, [ff, d, NE], synthetic_blocks(dt, NE * ff * d // blk[dt], 1 / np.sqrt(ff), rng)))

    def shexp():
        if not FS:
            return {}
        return {"ffn_gate_shexp.weight": mat(Q4_K, FS, d, s_d), "ffn_up_shexp.weight": mat(Q4_K, FS, d, s_d),
                "ffn_down_shexp.weight": mat(Q6_K, d, FS, 1 / np.sqrt(FS))}

    def dense():
        if not ND:
            return {}
        return {"ffn_gate.weight": mat(Q4_K, FD, d, s_d), "ffn_up.weight": mat(Q4_K, FD, d, s_d),
                "ffn_down.weight": mat(Q8_0, d, FD, 1 / np.sqrt(FD))}

    shared = (attn(), experts(), shexp(), dense()) if share else None
    for l in range(L):
        a_, ex, sh, dn = shared if share else (attn(), None, None, None)
        p = f"blk.{l}."
        T.update({p + k: v for k, v in a_.items()})
        T[p + "attn_norm.weight"] = f32(np.ones(d), [d])
        T[p + "ffn_norm.weight"] = f32(np.ones(d), [d])
        if l < ND:
            T.update({p + k: v for k, v in (dn if share else dense()).items()})
            continue
        T[p + "ffn_gate_inp.weight"] = f32(rng.standard_normal(NE * d) * (4.0 / np.sqrt(d)), [d, NE])
        g, u, dw = ex if share else experts()
        T[p + "ffn_gate_exps.weight"], T[p + "ffn_up_exps.weight"], T[p + "ffn_down_exps.weight"] = g, u, dw
        T.update({p + k: v for k, v in (sh if share else shexp()).items()})
    return hp, T


def stack_bytes_per_token(c: dict, n_layer: int | None = None) -> int:
    """Weight bytes one decode step reads: every layer's attention, the dense
    layers' FFN, per MoE layer the experts_used routed experts, the router and
    the shared FFN, then the head."""
    L = c["layers"] if n_layer is None else n_layer
    d, ff, H, KV, V, NE, NU = (c[k] for k in ("embd", "ff", "heads", "kv_heads", "vocab", "experts",
                                              "experts_used"))
    dt, FS, ND, FD = c["down_type"], c["shared_ff"], min(c["dense_layers"], L), c["dense_ff"]
    hd = d // H
    attn_b = tensor_bytes(Q4_K, (H + 2 * KV) * hd, d) + tensor_bytes(Q4_K, d, H * hd)
    expert_b = 2 * tensor_bytes(Q4_K, ff, d) + tensor_bytes(dt, d, ff)
    moe_b = NU * expert_b + NE * d * 4 + ((2 * tensor_bytes(Q4_K, FS, d) + tensor_bytes(Q6_K, d, FS)) if FS else 0)
    dense_b = (2 * tensor_bytes(Q4_K, FD, d) + tensor_bytes(Q8_0, d, FD)) if ND else 0
    return L * attn_b + ND * dense_b + (L - ND) * moe_b + tensor_bytes(Q6_K, V, d)
