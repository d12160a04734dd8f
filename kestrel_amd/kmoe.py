"""ctypes binding of libkmoe.so (include/kmoe.h) with torch tensors as device buffers.

The library is the product: if it is missing this module raises on import of
the binding; there is no CPU fallback. PyTorch only provides device memory and
the stream the calls are ordered on.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkmoe.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
REGIME_AVX2, REGIME_INT8, REGIME_EXACT = 0, 1, 2
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24),
         Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

STATUS = {0: "OK", -1: "INVALID", -2: "UNSUPPORTED", -3: "BUDGET", -4: "HIP", -5: "NOT_LOADED"}

class GpuMeasurements(C.Structure):
    """kmoe_gpu_measurements (include/kmoe.h)."""

    _fields_ = [("vram_total", C.c_uint64), ("vram_free", C.c_uint64), ("hbm_copy_bps", C.c_double),
                ("gemv_bps", C.c_double * 3), ("h2d_bps", C.c_double), ("d2h_bps", C.c_double),
                ("launch_s", C.c_double)]


class MoeDbg(C.Structure):
    """kmoe_moe_dbg (include/kmoe.h): device buffers of one captured moe_ffn."""

    _fields_ = [(n, C.c_void_p) for n in ("xq", "xd", "xs", "hq", "hd", "hs", "gate_sumi", "gate_mins", "up_sumi",
                                            "up_mins", "down_sumi", "down_mins")]


# Every symbol include/kmoe.h declares, with (restype, argtypes).
_P, _i32, _i64, _u32, _u64, _sz, _f = C.c_void_p, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_size_t, C.c_float
SIGNATURES = {
    "kmoe_create": (C.c_int, [C.c_int, C.POINTER(_P)]),
    "kmoe_destroy": (C.c_int, [_P]),
    "kmoe_last_error": (C.c_char_p, [_P]),
    "kmoe_abi_version": (C.c_int, []),
    "kmoe_set_stream": (C.c_int, [_P, _P]),
    "kmoe_use_own_stream": (C.c_int, [_P]),
    "kmoe_get_stream": (_P, [_P]),
    "kmoe_synchronize": (C.c_int, [_P]),
    "kmoe_set_regime": (C.c_int, [_P, C.c_int]),
    "kmoe_get_regime": (C.c_int, [_P]),
    "kmoe_workspace_generation": (C.c_int, [_P, C.POINTER(_u64)]),
    "kmoe_vram_set_limit": (C.c_int, [_P, _u64]),
    "kmoe_vram_usage": (C.c_int, [_P, C.POINTER(_u64), C.POINTER(_u64)]),
    "kmoe_device_alloc": (C.c_int, [_P, _sz, C.POINTER(_P)]),
    "kmoe_device_free": (C.c_int, [_P, _P]),
    "kmoe_copy_h2d": (C.c_int, [_P, _P, _P, _sz]),
    "kmoe_copy_d2h": (C.c_int, [_P, _P, _P, _sz]),
    "kmoe_matmul": (C.c_int, [_P, C.c_int, _P, _sz, _i64, _i64, _P, _i64, _P]),
    "kmoe_quantize_q8k": (C.c_int, [_P, _P, _i64, _i64, _P, _P, _P]),
    "kmoe_quantize_q8": (C.c_int, [_P, _P, _i64, _i64, _P, _P, _P]),
    "kmoe_q4k_block_sums": (C.c_int, [_P, _P, _i64, _i64, _P, _P, _i64, _P, _P]),
    "kmoe_q6k_block_sums": (C.c_int, [_P, _P, _i64, _i64, _P, _P, _i64, _P, _P]),
    "kmoe_q8_0_block_sums": (C.c_int, [_P, _P, _i64, _i64, _P, _i64, _P]),
    "kmoe_matvec_q8": (C.c_int, [_P, C.c_int, _P, _sz, _i64, _i64, _P, _P, _P, _i64, _P]),
    "kmoe_route": (C.c_int, [_P, _P, _i32, _i64, _P, _i64, _i32, _i32, _f, _P, _P, _P]),
    "kmoe_dispatch": (C.c_int, [_P, _P, _i64, _i32, _i32, _P, _P]),
    "kmoe_layer_create": (C.c_int, [_P, _u32, _P]),
    "kmoe_layer_destroy": (C.c_int, [_P, _u32]),
    "kmoe_router_upload": (C.c_int, [_P, _u32, _P, _sz]),
    "kmoe_expert_upload": (C.c_int, [_P, _u32, _u32, _i32, _P, _sz]),
    "kmoe_expert_upload_dev": (C.c_int, [_P, _u32, _u32, _i32, _P, _sz]),
    "kmoe_expert_upload_buf": (C.c_int, [_P, _u32, _u32, _P, _sz, C.POINTER(_u64)]),
    "kmoe_layer_preload": (C.c_int, [_P, _u32, C.POINTER(_P), C.POINTER(_u64), C.POINTER(_u64)]),
    "kmoe_expert_is_ready": (C.c_int, [_P, _u32, _u32]),
    "kmoe_expert_part": (C.c_int, [_P, _u32, _u32, _i32, C.POINTER(_P), C.POINTER(_sz)]),
    "kmoe_expert_read": (C.c_int, [_P, _u32, _u32, _i32, _P, _sz]),
    "kmoe_shared_expert_create": (C.c_int, [_P, _u32, _i64, _i32, _i32, _i32]),
    "kmoe_shared_expert_upload": (C.c_int, [_P, _u32, _i32, _P, _sz]),
    "kmoe_shared_gate_upload": (C.c_int, [_P, _u32, _P, _sz]),
    "kmoe_bytes_per_expert": (C.c_int, [_P, _u32, C.POINTER(_u64)]),
    "kmoe_moe_ffn": (C.c_int, [_P, _u32, _P, _i64, _P]),
    "kmoe_moe_ffn_dbg": (C.c_int, [_P, _u32, _P, _i64, _P, _P]),
    "kmoe_moe_ffn_host": (C.c_int, [_P, _u32, _P, _i64, _P]),
    "kmoe_moe_ffn_noalloc": (C.c_int, [_P, _u32, _P, _i64, _P]),
    "kmoe_matmul_host": (C.c_int, [_P, C.c_int, _P, _sz, _i64, _i64, _P, _i64, _P]),
    "kmoe_expert_part_layout": (C.c_int, [_P, _u32, _u32, _i32, C.POINTER(_i32)]),
    "kmoe_norm_matmul_rope_kv": (C.c_int, [_P, _P, _P, _P, _f, C.c_int, _P, _sz, _i64, _P, _P, _i32, _i32, _i32,
                                           _i32, _i64, _P, _P, _i32, _i64, _P, _P, _P, _P]),
    "kmoe_norm_moe_ffn": (C.c_int, [_P, _u32, _P, _P, _P, _f, _i64, _P, _P]),
    "kmoe_moe_last_routing": (C.c_int, [_P, _P, _P, _P, _P]),
    "kmoe_get_rows": (C.c_int, [_P, _i32, _P, _sz, _i64, _i64, _P, _i64, _P]),
    "kmoe_get_rows_dev": (C.c_int, [_P, _i32, _P, _sz, _i64, _i64, _P, _i64, _P]),
    "kmoe_rmsnorm": (C.c_int, [_P, _P, _P, _P, _i64, _i64, _f, _P]),
    "kmoe_norm_matmul": (C.c_int, [_P, _P, _P, _P, _f, C.c_int, _P, _sz, _i64, _i64, _i64, _P, _P]),
    "kmoe_rope": (C.c_int, [_P, _P, _i64, _i32, _i32, _i32, _i64, _P, _P, _i32]),
    "kmoe_kv_store": (C.c_int, [_P, _P, _P, _i64, _i64, _i64, _P, _i64, _P, _P]),
    "kmoe_attention": (C.c_int, [_P, _P, _P, _P, _i64, _i32, _i32, _i32, _i64, _P, _i64, _P]),
    "kmoe_attention_matmul": (C.c_int, [_P, _P, _P, _P, _i64, _i32, _i32, _i32, _i64, _P, _i64, _P, C.c_int, _P,
                                        _sz, _i64, _P]),
    "kmoe_rope_kv_store": (C.c_int, [_P, _P, _P, _P, _i64, _i32, _i32, _i32, _i32, _i64, _P, _P, _i32, _i64, _P,
                                     _P, _P]),
    "kmoe_swiglu": (C.c_int, [_P, _P, _P, _i64, _P]),
    "kmoe_add_rows": (C.c_int, [_P, _P, _P, _i64, _i64]),
    "kmoe_argmax": (C.c_int, [_P, _P, _i64, _P, _P, _i32]),
    "kmoe_pos_advance": (C.c_int, [_P, _P, _i32]),
    "kmoe_measure": (C.c_int, [_P, _P]),
    "kmoe_profile_enable": (C.c_int, [_P, C.c_int]),
    "kmoe_profile_read": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_double), C.POINTER(_i64)]),
}


class MoeDesc(C.Structure):
    """kmoe_moe_desc (include/kmoe.h)."""

    _fields_ = [
        ("n_expert", _u32),
        ("n_expert_used", _u32),
        ("norm_topk", _i32),
        ("weights_scale", _f),
        ("n_embd", _i64),
        ("n_ff", _i64),
        ("gate_type", _i32),
        ("up_type", _i32),
        ("down_type", _i32),
    ]


class KmoeError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"kmoe {STATUS.get(status, status)}: {msg}")
        self.status = status


_lib = None


def load_library(path: str = LIB_PATH):
    """Load libkmoe.so; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: run `python -m kestrel_amd.build` (or __graft_entry__.build())")
        L = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def bytes_for(t: int, n: int) -> int:
    bs, ts = BLOCK[t]
    if n % bs:
        raise ValueError(f"{n} not a multiple of block size {bs}")
    return n // bs * ts


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


class Context:
    """One device and one stream (torch's current stream unless `stream` is given)."""

    def __init__(self, device: int = 0, stream=None):
        import torch

        self.torch = torch
        self.lib = load_library()
        self.device = device
        self._descs = {}  # layer -> (n_expert, part lengths)
        h = _P()
        rc = self.lib.kmoe_create(device, C.byref(h))
        if rc != 0:
            raise KmoeError(rc, "kmoe_create failed")
        self.h = h
        s = stream if stream is not None else torch.cuda.current_stream(device)
        self.set_stream(s)

    def close(self):
        if getattr(self, "h", None):
            self.lib.kmoe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc: int):
        if rc != 0:
            raise KmoeError(rc, self.lib.kmoe_last_error(self.h).decode())

    def set_stream(self, stream):
        self.stream = stream
        self.check(self.lib.kmoe_set_stream(self.h, stream.cuda_stream))

    def sync(self):
        self.check(self.lib.kmoe_synchronize(self.h))

    def workspace_generation(self) -> int:
        """kmoe_workspace_generation: changes when a workspace is reallocated."""
        v = _u64()
        self.check(self.lib.kmoe_workspace_generation(self.h, C.byref(v)))
        return v.value

    def set_regime(self, regime: int):
        self.check(self.lib.kmoe_set_regime(self.h, regime))

    def vram_set_limit(self, limit: int):
        self.check(self.lib.kmoe_vram_set_limit(self.h, limit))

    def vram_usage(self):
        r, l = _u64(), _u64()
        self.check(self.lib.kmoe_vram_usage(self.h, C.byref(r), C.byref(l)))
        return r.value, l.value

    # ------------------------------------------------------------ kernel seam
    def _empty(self, shape, dtype):
        return self.torch.empty(shape, dtype=dtype, device=f"cuda:{self.device}")

    def matmul(self, t: int, w, rows: int, cols: int, x):
        """quant::matmul (quant.rs:229): x [S, cols] f32 -> [S, rows] f32."""
        x = x.reshape(-1, cols)
        out = self._empty((x.shape[0], rows), self.torch.float32)
        self.check(self.lib.kmoe_matmul(self.h, t, _ptr(w), w.numel() * w.element_size(), rows, cols, _ptr(x),
                                        x.shape[0], _ptr(out)))
        return out

    # ------------------------------------------------ rest of the decoder layer
    def get_rows(self, t: int, table, n_rows: int, cols: int, ids, out=None):
        """quant::get_row for token ids (host sequence, or a device uint32/int32 tensor)."""
        if hasattr(ids, "data_ptr"):
            s_rows = ids.numel()
            out = self._empty((s_rows, cols), self.torch.float32) if out is None else out
            self.check(self.lib.kmoe_get_rows_dev(self.h, t, _ptr(table), table.numel() * table.element_size(),
                                                  n_rows, cols, _ptr(ids), s_rows, _ptr(out)))
            return out
        a = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
        out = self._empty((a.size, cols), self.torch.float32) if out is None else out
        self.check(self.lib.kmoe_get_rows(self.h, t, _ptr(table), table.numel() * table.element_size(), n_rows,
                                          cols, a.ctypes.data, a.size, _ptr(out)))
        return out

    def rmsnorm(self, x, w, eps: float, y=None, out=None):
        """Transformer::rmsnorm over the last axis of x; with y, x += y first (in place)."""
        dim = w.numel()
        out = self.torch.empty_like(x) if out is None else out
        self.check(self.lib.kmoe_rmsnorm(self.h, _ptr(x), _ptr(y), _ptr(w), x.numel() // dim, dim, eps, _ptr(out)))
        return out

    def norm_matmul(self, x, norm_w, eps: float, t: int, w, rows: int, cols: int, y=None, h=None):
        """rmsnorm (x += y first when given) then quant::matmul of the normed rows: -> [S, rows]."""
        S = x.numel() // cols
        h = self._empty((S, cols), self.torch.float32) if h is None else h
        out = self._empty((S, rows), self.torch.float32)
        self.check(self.lib.kmoe_norm_matmul(self.h, _ptr(x), _ptr(y), _ptr(norm_w), eps, t, _ptr(w),
                                             w.numel() * w.element_size(), rows, cols, S, _ptr(h), _ptr(out)))
        return out

    def rope(self, x, n_heads: int, head_dim: int, rope_dim: int, pos0: int, inv_freq, neox: bool, pos_dev=None):
        """Transformer::rope in place on x [S, n_heads*head_dim]."""
        s_rows = x.numel() // (n_heads * head_dim)
        self.check(self.lib.kmoe_rope(self.h, _ptr(x), s_rows, n_heads, head_dim, rope_dim, pos0, _ptr(pos_dev),
                                      _ptr(inv_freq), int(neox)))
        return x

    def kv_store(self, k, v, kv_width: int, pos0: int, n_ctx: int, k_cache, v_cache, pos_dev=None):
        s_rows = k.numel() // kv_width
        self.check(self.lib.kmoe_kv_store(self.h, _ptr(k), _ptr(v), s_rows, kv_width, pos0, _ptr(pos_dev), n_ctx,
                                          _ptr(k_cache), _ptr(v_cache)))

    def norm_matmul_rope_kv(self, x, norm_w, eps: float, t: int, w, cols: int, n_head: int, n_kv: int,
                            head_dim: int, rope_dim: int, pos0: int, inv_freq, neox: bool, n_ctx: int, k_cache,
                            v_cache, y=None, pos_dev=None, h=None, qkv=None, q_out=None, x_out=None):
        """One token: norm_matmul over the q/k/v rows, then rope_kv_store of its parts; returns q_out.
        With x_out (another [1, cols] buffer) x + y goes there and x is left as it was."""
        rows = (n_head + 2 * n_kv) * head_dim
        h = self._empty((1, cols), self.torch.float32) if h is None else h
        qkv = self._empty((1, rows), self.torch.float32) if qkv is None else qkv
        q_out = self._empty((1, n_head * head_dim), self.torch.float32) if q_out is None else q_out
        self.check(self.lib.kmoe_norm_matmul_rope_kv(
            self.h, _ptr(x), _ptr(y), _ptr(norm_w), eps, t, _ptr(w), w.numel() * w.element_size(), cols, _ptr(h),
            _ptr(qkv), n_head, n_kv, head_dim, rope_dim, pos0, _ptr(pos_dev), _ptr(inv_freq), int(neox), n_ctx,
            _ptr(q_out), _ptr(k_cache), _ptr(v_cache), _ptr(x_out)))
        return q_out

    def rope_kv_store(self, q, k, v, n_head: int, n_kv: int, head_dim: int, rope_dim: int, pos0: int, inv_freq,
                      neox: bool, n_ctx: int, k_cache, v_cache, pos_dev=None, q_out=None):
        """RoPE of q (into q_out, returned) and k, then the f16 cache store of k and v."""
        s_rows = q.numel() // (n_head * head_dim)
        q_out = self._empty((s_rows, n_head * head_dim), self.torch.float32) if q_out is None else q_out
        self.check(self.lib.kmoe_rope_kv_store(self.h, _ptr(q), _ptr(k), _ptr(v), s_rows, n_head, n_kv, head_dim,
                                               rope_dim, pos0, _ptr(pos_dev), _ptr(inv_freq), int(neox), n_ctx,
                                               _ptr(q_out), _ptr(k_cache), _ptr(v_cache)))
        return q_out

    def attention(self, q, k_cache, v_cache, n_head: int, n_kv: int, head_dim: int, pos0: int, n_ctx: int,
                  pos_dev=None, out=None):
        """Transformer::attention: q [S, n_head*head_dim] -> [S, n_head*head_dim]."""
        s_rows = q.numel() // (n_head * head_dim)
        out = self._empty((s_rows, n_head * head_dim), self.torch.float32) if out is None else out
        self.check(self.lib.kmoe_attention(self.h, _ptr(q), _ptr(k_cache), _ptr(v_cache), s_rows, n_head, n_kv,
                                           head_dim, pos0, _ptr(pos_dev), n_ctx, _ptr(out)))
        return out

    def attention_matmul(self, q, k_cache, v_cache, n_head: int, n_kv: int, head_dim: int, pos0: int, n_ctx: int,
                         t: int, w, rows: int, pos_dev=None, attn=None):
        """Transformer::attention then self.mm(attn_output): -> [S, rows]."""
        s_rows = q.numel() // (n_head * head_dim)
        attn = self._empty((s_rows, n_head * head_dim), self.torch.float32) if attn is None else attn
        out = self._empty((s_rows, rows), self.torch.float32)
        self.check(self.lib.kmoe_attention_matmul(self.h, _ptr(q), _ptr(k_cache), _ptr(v_cache), s_rows, n_head, n_kv,
                                                  head_dim, pos0, _ptr(pos_dev), n_ctx, _ptr(attn), t, _ptr(w),
                                                  w.numel() * w.element_size(), rows, _ptr(out)))
        return out

    def swiglu(self, g, u, out=None):
        out = self.torch.empty_like(g) if out is None else out
        self.check(self.lib.kmoe_swiglu(self.h, _ptr(g), _ptr(u), g.numel(), _ptr(out)))
        return out

    def add_rows(self, x, b):
        cols = b.numel()
        self.check(self.lib.kmoe_add_rows(self.h, _ptr(x), _ptr(b), x.numel() // cols, cols))
        return x

    def argmax(self, logits, out=None, pos_dev=None, advance: int = 0):
        out = self._empty((1,), self.torch.int32) if out is None else out
        self.check(self.lib.kmoe_argmax(self.h, _ptr(logits), logits.numel(), _ptr(out), _ptr(pos_dev), advance))
        return out

    def pos_advance(self, pos_dev, by: int = 1):
        self.check(self.lib.kmoe_pos_advance(self.h, _ptr(pos_dev), by))

    def quantize_q8k(self, x):
        S, n = x.shape
        q = self._empty((S, n), self.torch.int8)
        d = self._empty((S, n // 256), self.torch.float32)
        bs = self._empty((S, n // 16), self.torch.int32)
        self.check(self.lib.kmoe_quantize_q8k(self.h, _ptr(x), S, n, _ptr(q), _ptr(d), _ptr(bs)))
        return q, d, bs

    def quantize_q8(self, x):
        S, n = x.shape
        q = self._empty((S, n), self.torch.int8)
        d = self._empty((S, n // 32), self.torch.float32)
        s16 = self._empty((S, n // 16), self.torch.int32)
        self.check(self.lib.kmoe_quantize_q8(self.h, _ptr(x), S, n, _ptr(q), _ptr(d), _ptr(s16)))
        return q, d, s16

    def matvec_q8(self, t, w, rows, cols, q, d, bs):
        S = q.shape[0]
        out = self._empty((S, rows), self.torch.float32)
        self.check(self.lib.kmoe_matvec_q8(self.h, t, _ptr(w), w.numel(), rows, cols, _ptr(q), _ptr(d), _ptr(bs), S,
                                           _ptr(out)))
        return out

    def q4k_block_sums(self, w, rows, cols, q, bs):
        S = q.shape[0]
        nb = cols // 256
        sumi = self._empty((S, rows, nb), self.torch.int32)
        mins = self._empty((S, rows, nb), self.torch.int32)
        self.check(self.lib.kmoe_q4k_block_sums(self.h, _ptr(w), rows, cols, _ptr(q), _ptr(bs), S, _ptr(sumi),
                                                _ptr(mins)))
        return sumi, mins

    def q6k_block_sums(self, w, rows, cols, q, bs):
        S = q.shape[0]
        nb = cols // 256
        sumi = self._empty((S, rows, nb), self.torch.int32)
        offs = self._empty((S, rows, nb), self.torch.int32)
        self.check(self.lib.kmoe_q6k_block_sums(self.h, _ptr(w), rows, cols, _ptr(q), _ptr(bs), S, _ptr(sumi),
                                                _ptr(offs)))
        return sumi, offs

    def q8_0_block_sums(self, w, rows, cols, q):
        S = q.shape[0]
        p = self._empty((S, rows, cols // 32), self.torch.int32)
        self.check(self.lib.kmoe_q8_0_block_sums(self.h, _ptr(w), rows, cols, _ptr(q), S, _ptr(p)))
        return p

    def route(self, router, h, k: int, norm_topk=True, weights_scale=0.0):
        E, d = router.shape
        S = h.shape[0]
        idx = self._empty((S, k), self.torch.int32)
        w = self._empty((S, k), self.torch.float32)
        logits = self._empty((S, E), self.torch.float32)
        self.check(self.lib.kmoe_route(self.h, _ptr(router), E, d, _ptr(h), S, k, int(norm_topk), weights_scale,
                                       _ptr(idx), _ptr(w), _ptr(logits)))
        return idx, w, logits

    def dispatch(self, idx, n_expert: int):
        S, k = idx.shape
        perm = self._empty((S * k,), self.torch.int32)
        off = self._empty((n_expert + 1,), self.torch.int32)
        self.check(self.lib.kmoe_dispatch(self.h, _ptr(idx), S, k, n_expert, _ptr(perm), _ptr(off)))
        return perm, off

    # ------------------------------------------------------------ expert tier
    def layer_create(self, layer: int, n_expert, n_used, d, ff, gate_type, up_type, down_type, norm_topk=True,
                     weights_scale=0.0):
        desc = MoeDesc(n_expert, n_used, int(norm_topk), weights_scale, d, ff, gate_type, up_type, down_type)
        self.check(self.lib.kmoe_layer_create(self.h, layer, C.byref(desc)))
        self._descs[layer] = (n_expert, (bytes_for(gate_type, d) * ff, bytes_for(up_type, d) * ff,
                                         bytes_for(down_type, ff) * d))

    def layer_destroy(self, layer: int):
        self.check(self.lib.kmoe_layer_destroy(self.h, layer))
        self._descs.pop(layer, None)

    def router_upload(self, layer: int, router: np.ndarray):
        r = np.ascontiguousarray(router, dtype=np.float32)
        self.check(self.lib.kmoe_router_upload(self.h, layer, r.ctypes.data, r.nbytes))

    def expert_upload(self, layer: int, e: int, part: int, data):
        if isinstance(data, np.ndarray):
            b = np.ascontiguousarray(data).view(np.uint8)
            self.check(self.lib.kmoe_expert_upload(self.h, layer, e, part, b.ctypes.data, b.nbytes))
        else:  # torch device tensor
            self.check(self.lib.kmoe_expert_upload_dev(self.h, layer, e, part, _ptr(data),
                                                       data.numel() * data.element_size()))

    def expert_upload_buf(self, layer: int, e: int, buf: np.ndarray, part_pos):
        """ExpertBuf (expert.rs:62-76): one host buffer with the expert's
        extents, part k at byte part_pos[k]; one host-to-device copy."""
        b = np.ascontiguousarray(buf).view(np.uint8)
        pos = (_u64 * 3)(*[int(p) for p in part_pos])
        self.check(self.lib.kmoe_expert_upload_buf(self.h, layer, e, b.ctypes.data, b.nbytes, pos))

    def layer_preload(self, layer: int, image: np.ndarray, part_off, part_stride) -> int:
        """ExpertStore::preload_all (expert.rs:620-641) from a model image in
        host memory (a mapped GGUF or KGUF): part k of expert e starts at byte
        part_off[k] + e * part_stride[k] of `image`. Returns the number of
        host-to-device copies (one per merged extent)."""
        img = np.ascontiguousarray(image).view(np.uint8)
        if layer not in self._descs:
            raise ValueError(f"layer {layer} not created by this context")
        n_expert, lens = self._descs[layer]
        for k, n in enumerate(lens):
            end = int(part_off[k]) + (n_expert - 1) * int(part_stride[k]) + n
            if int(part_off[k]) < 0 or int(part_stride[k]) < 0 or end > img.nbytes:
                raise ValueError(f"part {k}: expert extents end at {end} > image of {img.nbytes} bytes")
        base = (_P * 3)(*[img.ctypes.data + int(o) for o in part_off])
        stride = (_u64 * 3)(*[int(s) for s in part_stride])
        copies = _u64()
        self.check(self.lib.kmoe_layer_preload(self.h, layer, base, stride, C.byref(copies)))
        return copies.value

    def expert_is_ready(self, layer: int, e: int) -> bool:
        return self.lib.kmoe_expert_is_ready(self.h, layer, e) == 1

    def expert_part(self, layer: int, e: int, part: int):
        p, n = _P(), _sz()
        self.check(self.lib.kmoe_expert_part(self.h, layer, e, part, C.byref(p), C.byref(n)))
        return p.value, n.value

    def expert_read(self, layer: int, e: int, part: int) -> np.ndarray:
        """The part's GGUF bytes (ExpertBuf::part), whatever the tier's layout."""
        _, n = self.expert_part(layer, e, part)
        buf = np.empty(n, np.uint8)
        self.check(self.lib.kmoe_expert_read(self.h, layer, e, part, buf.ctypes.data, n))
        return buf

    def shared_expert(self, layer: int, n_ff: int, types, gate, up, down, gate_inp=None):
        """Attach a shared expert (transformer.rs:572-587): GGUF bytes (numpy
        uint8) of ffn_{gate,up,down}_shexp and the optional F32 gate vector."""
        self.check(self.lib.kmoe_shared_expert_create(self.h, layer, n_ff, *types))
        for p, b in enumerate((gate, up, down)):
            b = np.ascontiguousarray(b, dtype=np.uint8)
            self.check(self.lib.kmoe_shared_expert_upload(self.h, layer, p, b.ctypes.data, b.nbytes))
        if gate_inp is not None:
            g = np.ascontiguousarray(gate_inp, dtype=np.float32)
            self.check(self.lib.kmoe_shared_gate_upload(self.h, layer, g.ctypes.data, g.nbytes))

    def measure(self) -> dict:
        """kmoe_measure: the GPU figures kestrel's planner would otherwise estimate."""
        m = GpuMeasurements()
        self.check(self.lib.kmoe_measure(self.h, C.byref(m)))
        return {"vram_total": m.vram_total, "vram_free": m.vram_free, "hbm_copy_bps": m.hbm_copy_bps,
                "gemv_bps": {"Q4_K": m.gemv_bps[0], "Q6_K": m.gemv_bps[1], "Q8_0": m.gemv_bps[2]},
                "h2d_bps": m.h2d_bps, "d2h_bps": m.d2h_bps, "launch_s": m.launch_s}

    def bytes_per_expert(self, layer: int) -> int:
        v = _u64()
        self.check(self.lib.kmoe_bytes_per_expert(self.h, layer, C.byref(v)))
        return v.value

    def moe_ffn(self, layer: int, h, out=None):
        S, d = h.shape
        if out is None:
            out = self._empty((S, d), self.torch.float32)
        self.check(self.lib.kmoe_moe_ffn(self.h, layer, _ptr(h), S, _ptr(out)))
        return out

    def moe_ffn_dbg(self, layer: int, h, n_expert_used: int, n_ff: int, gate_type: int, down_type: int):
        """kmoe_moe_ffn_dbg: (out, dict of the captured device tensors): the
        int8 rows of h and of the SwiGLU output per slot (dispatch order), and
        the per-block integers [slots, rows, blocks] of gate, up and down."""
        t = self.torch
        S, d = h.shape
        slots, F = S * n_expert_used, n_ff
        bg, bd = (32 if gate_type == Q8_0 else 256), (32 if down_type == Q8_0 else 256)
        cap = dict(xq=self._empty((S, d), t.int8), xd=self._empty((S, d // bg), t.float32),
                   xs=self._empty((S, d // 16), t.int32), hq=self._empty((slots, F), t.int8),
                   hd=self._empty((slots, F // bd), t.float32), hs=self._empty((slots, F // 16), t.int32))
        for n in ("gate", "up"):
            for m in ("sumi", "mins"):
                cap[f"{n}_{m}"] = self._empty((slots, F, d // bg), t.int32)
        for m in ("sumi", "mins"):
            cap[f"down_{m}"] = self._empty((slots, d, F // bd), t.int32)
        out = self._empty((S, d), t.float32)
        dbg = MoeDbg(*[_ptr(cap[n]) for n, _ in MoeDbg._fields_])
        self.check(self.lib.kmoe_moe_ffn_dbg(self.h, layer, _ptr(h), S, _ptr(out), C.byref(dbg)))
        return out, cap

    def moe_ffn_host(self, layer: int, h: np.ndarray) -> np.ndarray:
        """kmoe_moe_ffn_host: host h [S, d] f32 in, host out back (synchronous)."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        out = np.empty_like(h)
        self.check(self.lib.kmoe_moe_ffn_host(self.h, layer, h.ctypes.data, h.shape[0], out.ctypes.data))
        return out

    def matmul_host(self, t: int, w, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
        """kmoe_matmul_host: x [S, cols] host f32; w host bytes (numpy) or a
        device tensor; returns out [S, rows] on the host (synchronous)."""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        out = np.empty((x.shape[0], rows), np.float32)
        if isinstance(w, np.ndarray):
            w = np.ascontiguousarray(w).view(np.uint8)
            wp, wn = w.ctypes.data, w.nbytes
        else:
            wp, wn = _ptr(w), w.numel() * w.element_size()
        self.check(self.lib.kmoe_matmul_host(self.h, t, wp, wn, rows, cols, x.ctypes.data, x.shape[0],
                                             out.ctypes.data))
        return out

    def expert_part_layout(self, layer: int, e: int, part: int) -> int:
        v = _i32()
        self.check(self.lib.kmoe_expert_part_layout(self.h, layer, e, part, C.byref(v)))
        return v.value

    def norm_moe_ffn(self, layer: int, x, norm_w, eps: float, y=None, f=None, out=None):
        """x += y (when given), f = rmsnorm(x) * norm_w, out = moe_ffn(f); returns out."""
        S, d = x.shape
        f = self._empty((S, d), self.torch.float32) if f is None else f
        if out is None:
            out = self._empty((S, d), self.torch.float32)
        self.check(self.lib.kmoe_norm_moe_ffn(self.h, layer, _ptr(x), _ptr(y), _ptr(norm_w), eps, S, _ptr(f),
                                              _ptr(out)))
        return out

    def last_routing(self, S: int, k: int, n_expert: int):
        idx = self._empty((S, k), self.torch.int32)
        w = self._empty((S, k), self.torch.float32)
        perm = self._empty((S * k,), self.torch.int32)
        off = self._empty((n_expert + 1,), self.torch.int32)
        self.check(self.lib.kmoe_moe_last_routing(self.h, _ptr(idx), _ptr(w), _ptr(perm), _ptr(off)))
        return idx, w, perm, off

    # ------------------------------------------------------------ profiling
    def profile_enable(self, on: bool = True):
        self.check(self.lib.kmoe_profile_enable(self.h, int(on)))

    def profile_read(self, kernel: str):
        ms, n = C.c_double(), _i64()
        self.check(self.lib.kmoe_profile_read(self.h, kernel.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value


@dataclass
class Shape:
    n_expert: int
    k: int
    d: int
    ff: int
    wtype: int
