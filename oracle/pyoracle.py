"""ctypes binding of the CPU oracle (test infrastructure only; see __init__.py)."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkmoe_oracle.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
REGIME_AVX2, REGIME_INT8, REGIME_EXACT = 0, 1, 2

_P = C.c_void_p
_i64 = C.c_int64
_sz = C.c_size_t


def build() -> str:
    """Compile the oracle in place (make); returns the library path."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class MoeLayer(C.Structure):
    """orc_moe_layer (kmoe_oracle.h)."""

    _fields_ = [
        ("n_expert", C.c_int32),
        ("n_expert_used", C.c_int32),
        ("norm_topk", C.c_int32),
        ("weights_scale", C.c_float),
        ("n_embd", C.c_int64),
        ("n_ff", C.c_int64),
        ("gate_type", C.c_int32),
        ("up_type", C.c_int32),
        ("down_type", C.c_int32),
        ("router", _P),
        ("gate", C.POINTER(_P)),
        ("up", C.POINTER(_P)),
        ("down", C.POINTER(_P)),
    ]


class SharedExpert(C.Structure):
    """orc_shared_expert (kmoe_oracle.h)."""

    _fields_ = [
        ("n_embd", C.c_int64),
        ("n_ff", C.c_int64),
        ("gate_type", C.c_int32),
        ("up_type", C.c_int32),
        ("down_type", C.c_int32),
        ("gate", _P),
        ("up", _P),
        ("down", _P),
        ("gate_inp", _P),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sig = {
            "orc_block_size": (_i64, [C.c_int]),
            "orc_type_size": (_i64, [C.c_int]),
            "orc_bytes_for": (_i64, [C.c_int, _i64]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_fill_normal": (None, [C.c_uint64, C.c_float, C.c_float, _P, _sz]),
            "orc_fill_xorshift_bytes": (None, [C.c_uint32, _P, _sz, C.c_uint8]),
            "orc_quantize_q8_0": (None, [_P, _sz, _P]),
            "orc_quantize_q4_k": (None, [_P, _sz, _P]),
            "orc_quantize_rows": (None, [C.c_int, _P, _sz, _sz, _P, C.c_int]),
            "orc_dequant_row": (C.c_int, [C.c_int, _P, _P, _sz]),
            "orc_q8row_quantize": (None, [_P, _sz, _P, _P, _P]),
            "orc_q8krow_quantize": (None, [_P, _sz, _P, _P, _P]),
            "orc_unpack": (C.c_int, [C.c_int, _P, _sz, _P, _P, _P]),
            "orc_dot_unpacked_scalar": (C.c_float, [_P, _P, _P, _sz, _P, _P, _P]),
            "orc_dot_unpacked_avx2": (C.c_float, [_P, _P, _P, _sz, _P, _P, _P]),
            "orc_dot_q8_0": (C.c_float, [_P, _sz, _P, _P]),
            "orc_dot_q4_0": (C.c_float, [_P, _sz, _P, _P]),
            "orc_dot_q4_k": (C.c_float, [_P, _sz, _P, _P, _P]),
            "orc_dot_q4_k_8k": (C.c_float, [_P, _sz, _P, _P, _P]),
            "orc_q4k_block_acc": (None, [_P, _sz, _P, _P, _P, _P]),
            "orc_q4k_block_acc_bruteforce": (None, [_P, _sz, _P, _P, _P, _P]),
            "orc_q8_0_block_acc": (None, [_P, _sz, _P, _P]),
            "orc_quantize_q6_k": (None, [_P, _sz, _P]),
            "orc_dot_q6_k_8k": (C.c_float, [_P, _sz, _P, _P, _P]),
            "orc_q6k_block_acc": (None, [_P, _sz, _P, _P, _P, _P]),
            "orc_q6k_block_acc_bruteforce": (None, [_P, _sz, _P, _P, _P]),
            "orc_quant_dot": (C.c_float, [_P, _P, _sz]),
            "orc_dot_f32": (C.c_float, [_P, _P, _sz]),
            "orc_gemm_f32": (None, [_P, _sz, _P, _sz, _sz, _P]),
            "orc_matmul": (C.c_int, [C.c_int, _P, _sz, _sz, _sz, _P, _sz, _P, C.c_int, C.c_int]),
            "orc_route": (C.c_int, [C.POINTER(MoeLayer), _P, _sz, _P, _P, C.c_int, C.c_int]),
            "orc_route_from_logits": (None, [_P, _sz, C.c_int, C.c_int, C.c_int, C.c_float, _P, _P]),
            "orc_dispatch": (None, [_P, _sz, C.c_int, C.c_int, _P, _P]),
            "orc_moe_ffn": (C.c_int, [C.POINTER(MoeLayer), _P, _sz, _P, C.c_int, C.c_int]),
            "orc_shared_expert_add": (C.c_int, [C.POINTER(SharedExpert), _P, _sz, _P, C.c_int, C.c_int]),
            "orc_f32_to_f16_n": (None, [_P, _P, _sz]),
            "orc_rmsnorm": (None, [_P, _P, _sz, _sz, C.c_float, _P]),
            "orc_rope_inv_freq": (None, [C.c_float, _sz, _P, _P]),
            "orc_rope": (None, [_P, _sz, _sz, _sz, _sz, _sz, _P, C.c_int]),
            "orc_attention": (None, [_P, _P, _P, _sz, _sz, _sz, _sz, _sz, _P]),
            "orc_argmax": (C.c_uint32, [_P, _sz]),
            "orc_swiglu": (None, [_P, _P, _sz, _P]),
            "orc_bench_gemv": (C.c_double, [C.c_int, _sz, _sz, _sz, C.c_int]),
            "orc_hw_threads": (C.c_int, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_P)


# ---------------------------------------------------------------- geometry
def block_size(t: int) -> int:
    return lib().orc_block_size(t)


def type_size(t: int) -> int:
    return lib().orc_type_size(t)


def bytes_for(t: int, n: int):
    v = lib().orc_bytes_for(t, n)
    return None if v < 0 else v


# ---------------------------------------------------------------- generators
def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(seed, mean, std, _p(out), n)
    return out


def xorshift_bytes(seed: int, n: int, mask: int = 0xFF) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().orc_fill_xorshift_bytes(seed, _p(out), n, mask)
    return out


def f16_bits(v: float) -> int:
    return lib().orc_f32_to_f16(v)


# ---------------------------------------------------------------- quantizers
def quantize(t: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """Quantize a [rows, cols] f32 matrix into GGUF row bytes of type t."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape if x.ndim == 2 else (1, x.shape[0])
    rb = bytes_for(t, cols)
    out = np.empty(rows * rb, dtype=np.uint8)
    lib().orc_quantize_rows(t, _p(x), rows, cols, _p(out), threads)
    return out


def dequant(t: int, w: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    rc = lib().orc_dequant_row(t, _p(np.ascontiguousarray(w, dtype=np.uint8)), _p(out), n)
    assert rc == 0
    return out


def q8k_quantize(x: np.ndarray):
    """Q8KRow::quantize per row of x [S, n] -> (q int8 [S,n], d f32 [S,n/256], bsums i32 [S,n/16])."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    S, n = x.shape
    q = np.empty((S, n), np.int8)
    d = np.empty((S, n // 256), np.float32)
    bs = np.empty((S, n // 16), np.int32)
    for s in range(S):
        lib().orc_q8krow_quantize(_p(x[s]), n, _p(q[s]), _p(d[s]), _p(bs[s]))
    return q, d, bs


def q8_quantize(x: np.ndarray):
    """Q8Row::quantize per row -> (q int8 [S,n], d f32 [S,n/32], s16 i32 [S,n/16])."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    S, n = x.shape
    q = np.empty((S, n), np.int8)
    d = np.empty((S, n // 32), np.float32)
    s16 = np.empty((S, n // 16), np.int32)
    for s in range(S):
        lib().orc_q8row_quantize(_p(x[s]), n, _p(q[s]), _p(d[s]), _p(s16[s]))
    return q, d, s16


def unpack(t: int, w: np.ndarray, n: int):
    q = np.empty(n, np.int8)
    sc = np.empty(n // 16, np.float32)
    mn = np.empty(n // 16, np.float32)
    rc = lib().orc_unpack(t, _p(np.ascontiguousarray(w, dtype=np.uint8)), n, _p(q), _p(sc), _p(mn))
    assert rc == 0
    return q, sc, mn


def q4k_block_acc(w_row: np.ndarray, n: int, q: np.ndarray, bsums: np.ndarray):
    nb = n // 256
    sumi = np.empty(nb, np.int32)
    mins = np.empty(nb, np.int32)
    lib().orc_q4k_block_acc(_p(w_row), n, _p(q), _p(bsums), _p(sumi), _p(mins))
    return sumi, mins


def q4k_block_acc_bruteforce(w_row: np.ndarray, n: int, q: np.ndarray, bsums: np.ndarray):
    nb = n // 256
    sumi = np.empty(nb, np.int64)
    mins = np.empty(nb, np.int64)
    lib().orc_q4k_block_acc_bruteforce(_p(w_row), n, _p(q), _p(bsums), _p(sumi), _p(mins))
    return sumi, mins


def q6k_block_acc(w_row: np.ndarray, n: int, q: np.ndarray, bsums: np.ndarray):
    nb = n // 256
    sumi = np.empty(nb, np.int32)
    offs = np.empty(nb, np.int32)
    lib().orc_q6k_block_acc(_p(w_row), n, _p(q), _p(bsums), _p(sumi), _p(offs))
    return sumi, offs


def q6k_block_acc_bruteforce(w_row: np.ndarray, n: int, q: np.ndarray):
    nb = n // 256
    sumi = np.empty(nb, np.int64)
    offs = np.empty(nb, np.int64)
    lib().orc_q6k_block_acc_bruteforce(_p(w_row), n, _p(q), _p(sumi), _p(offs))
    return sumi, offs


def q8_0_block_acc(w_row: np.ndarray, n: int, q: np.ndarray):
    p = np.empty(n // 32, np.int32)
    lib().orc_q8_0_block_acc(_p(w_row), n, _p(q), _p(p))
    return p


# ---------------------------------------------------------------- matmul / MoE
def matmul(t: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, regime: int = REGIME_AVX2,
           threads: int = 0) -> np.ndarray:
    """quant::matmul (quant.rs:229): x [S, cols] f32 -> out [S, rows] f32."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    S = x.shape[0]
    out = np.empty((S, rows), np.float32)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    rc = lib().orc_matmul(t, _p(w), w.nbytes, rows, cols, _p(x), S, _p(out), regime, threads)
    if rc != 0:
        raise ValueError(f"orc_matmul failed rc={rc}")
    return out


class Layer:
    """Owns the numpy buffers behind an orc_moe_layer."""

    def __init__(self, n_expert, n_used, d, ff, gate_type, up_type, down_type, router, gate, up, down,
                 norm_topk=True, weights_scale=0.0):
        self.router = np.ascontiguousarray(router, dtype=np.float32)
        self.gate = [np.ascontiguousarray(g, dtype=np.uint8) for g in gate]
        self.up = [np.ascontiguousarray(g, dtype=np.uint8) for g in up]
        self.down = [np.ascontiguousarray(g, dtype=np.uint8) for g in down]
        arr = _P * n_expert
        self._gp = arr(*[g.ctypes.data for g in self.gate])
        self._up = arr(*[g.ctypes.data for g in self.up])
        self._dp = arr(*[g.ctypes.data for g in self.down])
        self.c = MoeLayer(n_expert, n_used, int(norm_topk), weights_scale, d, ff, gate_type, up_type, down_type,
                          self.router.ctypes.data, self._gp, self._up, self._dp)
        self.n_expert, self.k, self.d, self.ff = n_expert, n_used, d, ff

    def route(self, h: np.ndarray, regime: int = REGIME_AVX2, threads: int = 0):
        h = np.ascontiguousarray(np.atleast_2d(h), dtype=np.float32)
        S = h.shape[0]
        idx = np.empty((S, self.k), np.uint32)
        w = np.empty((S, self.k), np.float32)
        rc = lib().orc_route(C.byref(self.c), _p(h), S, _p(idx), _p(w), regime, threads)
        assert rc == 0
        return idx, w

    def moe_ffn(self, h: np.ndarray, regime: int = REGIME_AVX2, threads: int = 0) -> np.ndarray:
        h = np.ascontiguousarray(np.atleast_2d(h), dtype=np.float32)
        S = h.shape[0]
        out = np.empty((S, self.d), np.float32)
        rc = lib().orc_moe_ffn(C.byref(self.c), _p(h), S, _p(out), regime, threads)
        if rc != 0:
            raise ValueError(f"orc_moe_ffn failed rc={rc}")
        return out


def shared_expert_add(out: np.ndarray, h: np.ndarray, d: int, ff: int, types, gate, up, down, gate_inp=None,
                      regime: int = REGIME_AVX2, threads: int = 0) -> np.ndarray:
    """transformer.rs:572-587 applied to a copy of out [S, d]; returns it."""
    h = np.ascontiguousarray(np.atleast_2d(h), dtype=np.float32)
    o = np.array(out, dtype=np.float32, copy=True).reshape(h.shape[0], d)
    bufs = [np.ascontiguousarray(b, dtype=np.uint8) for b in (gate, up, down)]
    gi = None if gate_inp is None else np.ascontiguousarray(gate_inp, dtype=np.float32)
    sx = SharedExpert(d, ff, types[0], types[1], types[2], bufs[0].ctypes.data, bufs[1].ctypes.data,
                      bufs[2].ctypes.data, None if gi is None else gi.ctypes.data)
    rc = lib().orc_shared_expert_add(C.byref(sx), _p(h), h.shape[0], _p(o), regime, threads)
    if rc != 0:
        raise ValueError(f"orc_shared_expert_add failed rc={rc}")
    return o


def route_from_logits(logits: np.ndarray, k: int, norm_topk=True, weights_scale=0.0):
    logits = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    S, E = logits.shape
    idx = np.empty((S, k), np.uint32)
    w = np.empty((S, k), np.float32)
    lib().orc_route_from_logits(_p(logits), S, E, k, int(norm_topk), weights_scale, _p(idx), _p(w))
    return idx, w


def dispatch(idx: np.ndarray, n_expert: int):
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    S, k = idx.shape
    perm = np.empty(S * k, np.uint32)
    offsets = np.empty(n_expert + 1, np.uint32)
    lib().orc_dispatch(_p(idx), S, k, n_expert, _p(perm), _p(offsets))
    return perm, offsets


def bench_gemv(t: int, rows: int, cols: int, iters: int, threads: int = 0) -> float:
    return lib().orc_bench_gemv(t, rows, cols, iters, threads)


def hw_threads() -> int:
    return lib().orc_hw_threads()


# ---------------------------------------------------------------- decoder layer
def f16_store(x: np.ndarray) -> np.ndarray:
    """half::f16::from_f32 per element (the KV cache store): uint16 bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Transformer::rmsnorm (transformer.rs:330-340) over the last axis."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    dim = w.size
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(w), x.size // dim, dim, eps, _p(out))
    return out


def rope_inv_freq(base: float, rope_dim: int, freqs=None) -> np.ndarray:
    out = np.empty(rope_dim // 2, np.float32)
    f = None if freqs is None else np.ascontiguousarray(freqs, dtype=np.float32)
    lib().orc_rope_inv_freq(base, rope_dim, None if f is None else _p(f), _p(out))
    return out


def rope(x: np.ndarray, n_heads: int, head_dim: int, rope_dim: int, pos0: int, inv_freq: np.ndarray,
         neox: bool) -> np.ndarray:
    """Transformer::rope (transformer.rs:342-358) on a copy of x [S, n_heads*head_dim]."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    S = y.size // (n_heads * head_dim)
    f = np.ascontiguousarray(inv_freq, dtype=np.float32)
    lib().orc_rope(_p(y), S, n_heads, head_dim, rope_dim, pos0, _p(f), int(neox))
    return y


def attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, n_head: int, n_kv: int, head_dim: int,
              pos0: int) -> np.ndarray:
    """Transformer::attention (transformer.rs:591-631); caches are uint16 f16
    bits [positions, n_kv*head_dim] holding at least pos0 + S rows."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    S = q.size // (n_head * head_dim)
    kc = np.ascontiguousarray(k_cache, dtype=np.uint16)
    vc = np.ascontiguousarray(v_cache, dtype=np.uint16)
    assert kc.size >= (pos0 + S) * n_kv * head_dim and vc.size == kc.size
    out = np.empty((S, n_head * head_dim), np.float32)
    lib().orc_attention(_p(q), _p(kc), _p(vc), S, n_head, n_kv, head_dim, pos0, _p(out))
    return out


def argmax(logits: np.ndarray) -> int:
    l = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    return int(lib().orc_argmax(_p(l), l.size))


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


class Transformer:
    """Transformer::forward (transformer.rs:278-302, 375-467) restated over
    the oracle's kernels, for parity tests of whole decode stacks.

    hp: arch ("llama" rotates pairs (2i, 2i+1), the others (i, i + rd/2)),
    n_layer, n_embd, n_head, n_head_kv, head_dim, rope_dim, rope_freq_base,
    rms_eps, n_ctx, n_batch; MoE models add n_expert, n_expert_used,
    norm_topk, weights_scale. tensors: GGUF name -> (ggml type, dims with the
    contiguous dimension first, uint8 bytes)."""

    def __init__(self, hp: dict, tensors: dict, regime: int = REGIME_AVX2, threads: int = 0):
        self.hp, self.t, self.regime, self.threads = hp, tensors, regime, threads
        self.d, self.nh, self.nkv, self.hd = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        self.neox = hp["arch"] != "llama"
        self.n_ctx = hp["n_ctx"]
        freqs = self.vec("rope_freqs.weight") if "rope_freqs.weight" in tensors else None
        self.inv_freq = rope_inv_freq(hp["rope_freq_base"], hp["rope_dim"], freqs)
        kvw = self.nkv * self.hd
        self.k_cache = [np.zeros((self.n_ctx, kvw), np.uint16) for _ in range(hp["n_layer"])]
        self.v_cache = [np.zeros((self.n_ctx, kvw), np.uint16) for _ in range(hp["n_layer"])]
        self.cached = 0
        self.moe = {}
        for l in range(hp["n_layer"]):
            p = f"blk.{l}."
            if p + "ffn_gate_exps.weight" not in tensors:
                continue
            E = hp["n_expert"]
            parts = []
            for name in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
                ty, dims, b = tensors[p + name + ".weight"]
                parts.append((ty, np.split(np.ascontiguousarray(b, dtype=np.uint8), E)))
            ff = tensors[p + "ffn_gate_exps.weight"][1][1]
            router = self.vec(p + "ffn_gate_inp.weight").reshape(E, self.d)
            self.moe[l] = Layer(E, hp["n_expert_used"], self.d, ff, parts[0][0], parts[1][0], parts[2][0], router,
                                parts[0][1], parts[1][1], parts[2][1], hp.get("norm_topk", True),
                                hp.get("weights_scale", 0.0))

    def vec(self, name: str) -> np.ndarray:
        ty, dims, b = self.t[name]
        return dequant(ty, b, int(np.prod(dims)))

    def mm(self, name: str, x: np.ndarray) -> np.ndarray:
        ty, dims, b = self.t[name]
        return matmul(ty, b, int(np.prod(dims[1:])), dims[0], x, self.regime, self.threads)

    def forward(self, tokens) -> np.ndarray:
        tokens = list(tokens)
        if not tokens:
            raise ValueError("forward() needs at least one token")
        if self.cached + len(tokens) > self.n_ctx:
            raise ValueError("context full")
        n_batch = max(1, self.hp.get("n_batch", 512))
        logits = None
        for i in range(0, len(tokens), n_batch):
            logits = self._chunk(tokens[i:i + n_batch])
        return logits

    def _chunk(self, tokens) -> np.ndarray:
        hp, d, nh, nkv, hd = self.hp, self.d, self.nh, self.nkv, self.hd
        S, pos0, eps = len(tokens), self.cached, hp["rms_eps"]
        ety, edims, eb = self.t["token_embd.weight"]
        rb = bytes_for(ety, d)
        x = np.empty((S, d), np.float32)
        for s, tok in enumerate(tokens):
            if tok >= edims[1]:
                raise ValueError(f"token id {tok} out of range")
            x[s] = dequant(ety, eb[tok * rb:(tok + 1) * rb], d)
        kvw = nkv * hd
        for l in range(hp["n_layer"]):
            p = f"blk.{l}."
            h = rmsnorm(x, self.vec(p + "attn_norm.weight"), eps)
            q, k, v = (self.mm(p + f"attn_{n}.weight", h) for n in ("q", "k", "v"))
            for n, y in (("q", q), ("k", k), ("v", v)):
                if p + f"attn_{n}.bias" in self.t:
                    y += self.vec(p + f"attn_{n}.bias")[None, :]
            if p + "attn_q_norm.weight" in self.t:
                q = rmsnorm(q.reshape(-1, hd), self.vec(p + "attn_q_norm.weight"), eps).reshape(S, nh * hd)
            if p + "attn_k_norm.weight" in self.t:
                k = rmsnorm(k.reshape(-1, hd), self.vec(p + "attn_k_norm.weight"), eps).reshape(S, kvw)
            q = rope(q, nh, hd, hp["rope_dim"], pos0, self.inv_freq, self.neox)
            k = rope(k, nkv, hd, hp["rope_dim"], pos0, self.inv_freq, self.neox)
            self.k_cache[l][pos0:pos0 + S] = f16_store(k)
            self.v_cache[l][pos0:pos0 + S] = f16_store(v)
            ctx = attention(q, self.k_cache[l], self.v_cache[l], nh, nkv, hd, pos0)
            x = x + self.mm(p + "attn_output.weight", ctx)
            h = rmsnorm(x, self.vec(p + "ffn_norm.weight"), eps)
            if l in self.moe:
                y = self.moe[l].moe_ffn(h, self.regime, self.threads)
                if p + "ffn_gate_shexp.weight" in self.t:
                    ts = [self.t[p + f"ffn_{n}_shexp.weight"] for n in ("gate", "up", "down")]
                    gi = self.vec(p + "ffn_gate_inp_shexp.weight") if p + "ffn_gate_inp_shexp.weight" in self.t \
                        else None
                    y = shared_expert_add(y, h, d, ts[0][1][1], [t[0] for t in ts], ts[0][2], ts[1][2], ts[2][2],
                                          gi, self.regime, self.threads)
            else:
                g = self.mm(p + "ffn_gate.weight", h)
                u = self.mm(p + "ffn_up.weight", h)
                y = self.mm(p + "ffn_down.weight", swiglu(g, u))
            x = x + y
        self.cached += S
        normed = rmsnorm(x[S - 1:S], self.vec("output_norm.weight"), eps)
        head = "output.weight" if "output.weight" in self.t else "token_embd.weight"
        return self.mm(head, normed)[0]
