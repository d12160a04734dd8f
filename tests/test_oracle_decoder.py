"""Pins for the oracle's restatement of the rest of the decoder layer
(transformer.rs:216-226, 330-358, 411-418, 591-631; sampler.rs:104-112).

Each check uses a formulation independent of the oracle's loops: float64
numpy / scipy, complex rotations for RoPE, numpy's float16 rounding for the
KV store, invariants (relative-position dependence of rotated dot products,
attention over one position returns v) that a dropped term, a flipped sign or
a transposed head mapping would break."""
import numpy as np
import pytest
from scipy.special import softmax

from oracle import pyoracle as orc


def test_rmsnorm_matches_float64_formula():
    rng = np.random.default_rng(1)
    for dim, eps in [(64, 1e-5), (2048, 1e-6), (4096, 1e-5)]:
        x = (rng.standard_normal((5, dim)) * 3).astype(np.float32)
        w = rng.standard_normal(dim).astype(np.float32)
        got = orc.rmsnorm(x, w, eps)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * w
        assert np.abs(got - ref).max() <= 2e-6 * np.abs(ref).max(), dim
    # eps dominates a zero row: out = 0, no NaN
    assert np.all(orc.rmsnorm(np.zeros((1, 64), np.float32), np.ones(64, np.float32), 1e-5) == 0)


@pytest.mark.parametrize("base,rd", [(10000.0, 128), (1e6, 64), (500000.0, 96)])
def test_rope_frequencies(base, rd):
    f = orc.rope_inv_freq(base, rd)
    # the exponent is an f32 quotient (transformer.rs:217); the power is exact here
    e32 = (-(2.0 * np.arange(rd // 2, dtype=np.float32)) / np.float32(rd)).astype(np.float32)
    ref = np.float64(np.float32(base)) ** e32.astype(np.float64)
    assert f[0] == 1.0
    assert np.allclose(f, ref, rtol=1.2e-7, atol=0)
    scale = np.linspace(1.0, 8.0, rd // 2).astype(np.float32)  # rope_freqs.weight divides
    assert np.allclose(orc.rope_inv_freq(base, rd, scale), ref / scale, rtol=5e-7, atol=0)


def _rope_complex(x, n_heads, hd, rd, pos0, inv_freq, neox):
    """Rotation of each pair as multiplication by exp(i * pos * theta) in float64."""
    S = x.shape[0]
    y = x.astype(np.float64).reshape(S, n_heads, hd).copy()
    half = rd // 2
    a = np.arange(half) if neox else 2 * np.arange(half)
    b = a + half if neox else a + 1
    pos = (pos0 + np.arange(S)).astype(np.float32)[:, None]
    ang = (pos * inv_freq[None, :].astype(np.float32)).astype(np.float64)  # the f32 angle
    z = (y[:, :, a] + 1j * y[:, :, b]) * np.exp(1j * ang)[:, None, :]
    y[:, :, a], y[:, :, b] = z.real, z.imag
    return y.reshape(S, n_heads * hd)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("hd,rd", [(128, 128), (64, 32)])
def test_rope_is_the_complex_rotation(neox, hd, rd):
    rng = np.random.default_rng(2)
    nh, S, pos0 = 4, 6, 37
    x = rng.standard_normal((S, nh * hd)).astype(np.float32)
    f = orc.rope_inv_freq(10000.0, rd)
    got = orc.rope(x, nh, hd, rd, pos0, f, neox)
    ref = _rope_complex(x, nh, hd, rd, pos0, f, neox)
    assert np.abs(got - ref).max() < 2e-6 * np.abs(ref).max()
    # dims past rope_dim are untouched; position 0 is the identity
    r = got.reshape(S, nh, hd)
    assert np.array_equal(r[:, :, rd:], x.reshape(S, nh, hd)[:, :, rd:])
    assert np.array_equal(orc.rope(x[:1], nh, hd, rd, 0, f, neox), x[:1])


def test_rope_scores_depend_on_relative_position_only():
    rng = np.random.default_rng(3)
    hd = 64
    q = rng.standard_normal((1, hd)).astype(np.float32)
    k = rng.standard_normal((1, hd)).astype(np.float32)
    f = orc.rope_inv_freq(10000.0, hd)
    dots = []
    for m in (5, 105, 1005):
        qr = orc.rope(q, 1, hd, hd, m + 3, f, True).astype(np.float64)
        kr = orc.rope(k, 1, hd, hd, m, f, True).astype(np.float64)
        dots.append(float(qr @ kr.T))
    assert np.allclose(dots, dots[0], rtol=2e-4, atol=1e-4), dots


def test_kv_store_rounds_like_numpy_float16():
    rng = np.random.default_rng(4)
    x = np.concatenate([
        rng.standard_normal(4096).astype(np.float32),
        np.array([65504.0, 65520.0, 1e6, -1e6, 6e-8, 3e-8, 1e-9, 0.0, -0.0, np.inf, -np.inf], np.float32),
        # exact ties between two f16 values: round to even
        (np.arange(1, 200, dtype=np.float32) * 2.0 ** -11 + 1.0),
    ])
    got = orc.f16_store(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def _attention_float64(q, kc, vc, nh, nkv, hd, pos0):
    S = q.shape[0]
    kf = kc.view(np.float16).astype(np.float64).reshape(-1, nkv, hd)
    vf = vc.view(np.float16).astype(np.float64).reshape(-1, nkv, hd)
    out = np.zeros((S, nh, hd))
    qq = q.astype(np.float64).reshape(S, nh, hd)
    for s in range(S):
        n = pos0 + s + 1
        for h in range(nh):
            g = h // (nh // nkv)
            sc = kf[:n, g, :] @ qq[s, h] / np.sqrt(hd)
            out[s, h] = softmax(sc) @ vf[:n, g, :]
    return out.reshape(S, nh * hd)


@pytest.mark.parametrize("nh,nkv,hd,pos0,S", [(4, 4, 64, 0, 3), (8, 2, 64, 70, 2), (4, 1, 128, 130, 1)])
def test_attention_matches_float64_softmax(nh, nkv, hd, pos0, S):
    rng = np.random.default_rng(nh + pos0)
    n = pos0 + S
    kc = orc.f16_store(rng.standard_normal((n, nkv * hd)) * 2)
    vc = orc.f16_store(rng.standard_normal((n, nkv * hd)))
    q = rng.standard_normal((S, nh * hd)).astype(np.float32)
    got = orc.attention(q, kc, vc, nh, nkv, hd, pos0)
    ref = _attention_float64(q, kc, vc, nh, nkv, hd, pos0)
    assert np.abs(got - ref).max() < 1e-5 * max(1.0, np.abs(ref).max())


def test_attention_invariants():
    rng = np.random.default_rng(5)
    nh, nkv, hd = 4, 2, 64
    kc = orc.f16_store(rng.standard_normal((3, nkv * hd)))
    vc = orc.f16_store(rng.standard_normal((3, nkv * hd)))
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    # one visible position: every head returns its kv head's v exactly
    out = orc.attention(q, kc, vc, nh, nkv, hd, 0).reshape(nh, hd)
    v0 = vc[0].view(np.float16).astype(np.float32).reshape(nkv, hd)
    for h in range(nh):
        assert np.array_equal(out[h], v0[h // 2]), h
    # causality: positions after the query's do not matter
    a = orc.attention(q, kc, vc, nh, nkv, hd, 1)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[2], vc2[2] = 0x3C00, 0x4000
    assert np.array_equal(a, orc.attention(q, kc2, vc2, nh, nkv, hd, 1))


def test_argmax_first_of_ties_and_nan():
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax(np.array([-np.inf, -1], np.float32)) == 1
    assert orc.argmax(np.array([0, np.nan, 5, 5], np.float32)) == 2
    assert orc.argmax(np.array([np.nan, 1, 2], np.float32)) == 0  # every comparison with NaN fails
    x = np.random.default_rng(6).standard_normal(32000).astype(np.float32)
    assert orc.argmax(x) == int(np.argmax(x))


def _f32_model(rng, arch, n_layer, d, nh, nkv, hd, ff, vocab, bias, qk_norm, rope_dim):
    """A dense decoder with F32 weights: hp, tensors (GGUF names) and the same
    weights as float64 arrays."""
    W, T = {}, {}

    def add(name, a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        W[name] = a.astype(np.float64)
        dims = [a.shape[-1]] + ([a.shape[0]] if a.ndim == 2 else [])
        T[name] = (0, dims, a.view(np.uint8).reshape(-1))

    add("token_embd.weight", rng.standard_normal((vocab, d)))
    add("output_norm.weight", 1 + 0.1 * rng.standard_normal(d))
    add("output.weight", 0.05 * rng.standard_normal((vocab, d)))
    for l in range(n_layer):
        p = f"blk.{l}."
        add(p + "attn_norm.weight", 1 + 0.1 * rng.standard_normal(d))
        add(p + "ffn_norm.weight", 1 + 0.1 * rng.standard_normal(d))
        add(p + "attn_q.weight", 0.08 * rng.standard_normal((nh * hd, d)))
        add(p + "attn_k.weight", 0.08 * rng.standard_normal((nkv * hd, d)))
        add(p + "attn_v.weight", 0.05 * rng.standard_normal((nkv * hd, d)))
        add(p + "attn_output.weight", 0.05 * rng.standard_normal((d, nh * hd)))
        if bias:
            for n, w in (("q", nh * hd), ("k", nkv * hd), ("v", nkv * hd)):
                add(p + f"attn_{n}.bias", 0.1 * rng.standard_normal(w))
        if qk_norm:
            add(p + "attn_q_norm.weight", 1 + 0.1 * rng.standard_normal(hd))
            add(p + "attn_k_norm.weight", 1 + 0.1 * rng.standard_normal(hd))
        add(p + "ffn_gate.weight", 0.05 * rng.standard_normal((ff, d)))
        add(p + "ffn_up.weight", 0.05 * rng.standard_normal((ff, d)))
        add(p + "ffn_down.weight", 0.05 * rng.standard_normal((d, ff)))
    hp = dict(arch=arch, n_layer=n_layer, n_embd=d, n_head=nh, n_head_kv=nkv, head_dim=hd, rope_dim=rope_dim,
              rope_freq_base=10000.0, rms_eps=1e-5, n_ctx=64, n_batch=5)
    return hp, T, W


class _Float64Decoder:
    """forward_chunk_inner (transformer.rs:375-467) written out in float64
    numpy: matrix products, complex rotations for RoPE, scipy's softmax, the
    KV history kept as float16 (the cache's precision)."""

    def __init__(self, hp, W):
        self.hp, self.W = hp, W
        self.kc = [[] for _ in range(hp["n_layer"])]
        self.vc = [[] for _ in range(hp["n_layer"])]
        rd = hp["rope_dim"]
        e32 = (-(2.0 * np.arange(rd // 2, dtype=np.float32)) / np.float32(rd)).astype(np.float32)
        self.inv = np.float64(np.float32(hp["rope_freq_base"])) ** e32.astype(np.float64)
        self.pos = 0

    def norm(self, x, w):
        return x / np.sqrt((x ** 2).mean(axis=-1, keepdims=True) + self.hp["rms_eps"]) * w

    def rope(self, x, n_heads, pos):
        hd, rd = self.hp["head_dim"], self.hp["rope_dim"]
        y = x.reshape(n_heads, hd).copy()
        half = rd // 2
        a = np.arange(half) if self.hp["arch"] != "llama" else 2 * np.arange(half)
        b = a + half if self.hp["arch"] != "llama" else a + 1
        z = (y[:, a] + 1j * y[:, b]) * np.exp(1j * pos * self.inv)[None, :]
        y[:, a], y[:, b] = z.real, z.imag
        return y.reshape(-1)

    def forward(self, tokens):
        hp, W = self.hp, self.W
        nh, nkv, hd = hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        for tok in tokens:  # one row at a time: causal attention makes rows independent of later ones
            x = W["token_embd.weight"][tok].copy()
            for l in range(hp["n_layer"]):
                p = f"blk.{l}."
                h = self.norm(x, W[p + "attn_norm.weight"])
                q, k, v = (W[p + f"attn_{n}.weight"] @ h for n in "qkv")
                if p + "attn_q.bias" in W:
                    q, k, v = q + W[p + "attn_q.bias"], k + W[p + "attn_k.bias"], v + W[p + "attn_v.bias"]
                if p + "attn_q_norm.weight" in W:
                    q = self.norm(q.reshape(nh, hd), W[p + "attn_q_norm.weight"]).reshape(-1)
                    k = self.norm(k.reshape(nkv, hd), W[p + "attn_k_norm.weight"]).reshape(-1)
                q, k = self.rope(q, nh, self.pos), self.rope(k, nkv, self.pos)
                self.kc[l].append(k.astype(np.float16).astype(np.float64))
                self.vc[l].append(v.astype(np.float16).astype(np.float64))
                K = np.stack(self.kc[l]).reshape(-1, nkv, hd)
                V = np.stack(self.vc[l]).reshape(-1, nkv, hd)
                att = np.empty(nh * hd)
                for hh in range(nh):
                    g = hh // (nh // nkv)
                    att[hh * hd:(hh + 1) * hd] = softmax(K[:, g, :] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)) @ V[:, g, :]
                x = x + W[p + "attn_output.weight"] @ att
                h = self.norm(x, W[p + "ffn_norm.weight"])
                gte, up = W[p + "ffn_gate.weight"] @ h, W[p + "ffn_up.weight"] @ h
                x = x + W[p + "ffn_down.weight"] @ (gte / (1 + np.exp(-gte)) * up)
            self.pos += 1
        return W["output.weight"] @ self.norm(x, W["output_norm.weight"])


@pytest.mark.parametrize("arch,bias,qk_norm,nkv,rope_dim", [("llama", False, False, 2, 64), ("qwen2", True, False, 1, 32),
                                                           ("qwen3", False, True, 4, 64)])
def test_transformer_composition_matches_float64(arch, bias, qk_norm, nkv, rope_dim):
    """The oracle's Transformer (the composition of the pinned parts, in
    forward_chunk_inner's order) against the same decoder written out in
    float64, on F32 weights in the exact regime: a prompt chunked by n_batch
    and then single tokens, every logit within 1e-4 of the scale."""
    rng = np.random.default_rng(len(arch) + nkv)
    hp, T, W = _f32_model(rng, arch, 2, 128, 4, nkv, 64, 256, 300, bias, qk_norm, rope_dim)
    ref = orc.Transformer(hp, T, regime=orc.REGIME_EXACT)
    f64 = _Float64Decoder(hp, W)
    for toks in ([3, 17, 5, 99, 250, 7, 1, 2], [11], [200], [0]):
        a, b = ref.forward(toks), f64.forward(toks)
        assert np.abs(a - b).max() <= 1e-4 * max(1.0, np.abs(b).max()), (arch, len(toks), np.abs(a - b).max())
