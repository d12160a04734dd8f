"""Integer parity inside kmoe_moe_ffn: the per-block accumulators of the
kernels that produce the layer's output, bit for bit against the oracle.

kmoe_moe_ffn_dbg runs the same kernels as kmoe_moe_ffn (the single-token
tiled gate/up and split-K down kernels, the few-rows kernels, the int8
matrix-core kernels, the register and LDS-staged kernels) and also returns
what they computed on the integer side:
  - the int8 rows of h the gate/up products read (Q8KRow / Q8Row::quantize,
    qdot.rs:30-49, :347-367), checked against the oracle's quantization;
  - per (slot, row, block) the integers of dot_q4_k_8k (sumi, mins;
    avx2.rs:361-374), dot_q6_k_8k (sumi, offs; :398-414) and dot_q8_0 (p;
    :49-58), checked against the oracle's per-row accumulators on the same
    int8 inputs: x's rows for gate/up, and the kernel's own int8 rows of the
    SwiGLU output for down (those follow from an f32 h whose epilogue sums in
    another order, so the oracle is given the same int8 rows).
Slots of experts the regime sends to the f32 path (AVX2 regime, >= 4 rows,
quant.rs:242-260) have no integers and read 0.
"""
import numpy as np
import pytest

from tests.helpers import Q4_K, Q6_K, Q8_0, LayerSpec, rel_l2, row_bytes

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def ctx():
    import torch

    from kestrel_amd.kmoe import Context

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    c = Context(0)
    yield c
    c.sync()
    c.close()


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def oracle_ints(orc, t, w, rows, cols, q, bs):
    """The oracle's per-block integers of every row of W [rows, cols] (GGUF
    bytes) against one int8 activation row."""
    rb = row_bytes(t, cols)
    nb = cols // (32 if t == Q8_0 else 256)
    s = np.empty((rows, nb), np.int32)
    m = np.zeros((rows, nb), np.int32)
    for r in range(rows):
        row = w[r * rb:(r + 1) * rb]
        if t == Q4_K:
            s[r], m[r] = orc.q4k_block_acc(row, cols, q, bs)
        elif t == Q6_K:
            s[r], m[r] = orc.q6k_block_acc(row, cols, q, bs)
        else:
            s[r] = orc.q8_0_block_acc(row, cols, q)
    return s, m


def plant_extremes(w: np.ndarray, t: int):
    """Every 5th block all 0xFF (largest nibbles, 6-bit scales and mins 63,
    Q6_K's high bits and most negative scale byte, Q8_0's -1 weights with a
    NaN-free f16 scale kept), next to the random ones."""
    bs = {Q4_K: 144, Q6_K: 210, Q8_0: 34}[t]
    blk = w.reshape(-1, bs)
    keep = {Q4_K: slice(0, 4), Q6_K: slice(208, 210), Q8_0: slice(0, 2)}[t]
    saved = blk[::5, keep].copy()
    blk[::5] = 0xFF
    blk[::5, keep] = saved


_lid = [500]


def run_capture(ctx, orc, spec: LayerSpec, S: int, regime: int, h: np.ndarray):
    lid = _lid[0]
    _lid[0] += 1
    spec.upload(ctx, lid)
    try:
        ctx.set_regime(regime)
        out, cap = ctx.moe_ffn_dbg(lid, dev(h), spec.k, spec.ff, spec.gate_type, spec.down_type)
        cap = {n: host(v) for n, v in cap.items()}
        out = host(out)
        idx, w, perm, off = (host(t) for t in ctx.last_routing(S, spec.k, spec.n_expert))
        plain = host(ctx.moe_ffn(lid, dev(h)))
    finally:
        ctx.set_regime(0)
        ctx.layer_destroy(lid)
    assert np.array_equal(out.view(np.uint32), plain.view(np.uint32)), "capture changed the output bits"
    return out, cap, idx.view(np.uint32).reshape(-1), perm.view(np.uint32), off.view(np.uint32)


def check_ints(orc, spec: LayerSpec, S: int, regime: int, h: np.ndarray, out, cap, idx, perm, off):
    d, F, k = spec.d, spec.ff, spec.k
    L = spec.oracle_layer()
    ridx, _ = L.route(h, regime)
    assert np.array_equal(idx, ridx.reshape(-1)), "routing differs"
    gq = orc.q8_quantize if spec.gate_type == Q8_0 else orc.q8k_quantize
    xq, xd, xs = gq(h)
    counts = np.diff(off.astype(np.int64))
    int_slots = 0
    for p in range(S * k):
        flat = int(perm[p])
        s, e = flat // k, int(idx[flat])
        on_int = regime == 1 or (regime == 0 and counts[e] < 4)
        if not on_int:
            for n in ("gate_sumi", "gate_mins", "up_sumi", "up_mins", "down_sumi", "down_mins"):
                assert not cap[n][p].any(), (n, p)
            continue
        int_slots += 1
        assert np.array_equal(cap["xq"][s], xq[s]) and np.array_equal(cap["xs"][s], xs[s])
        assert np.array_equal(cap["xd"][s].view(np.uint32), xd[s].view(np.uint32))
        for part, wb, t in (("gate", spec.gate[e], spec.gate_type), ("up", spec.up[e], spec.up_type)):
            es, em = oracle_ints(orc, t, wb, F, d, xq[s], xs[s])
            assert np.array_equal(cap[f"{part}_sumi"][p], es), (part, p, e)
            if t != Q8_0:
                assert np.array_equal(cap[f"{part}_mins"][p], em), (part, p, e)
        es, em = oracle_ints(orc, spec.down_type, spec.down[e], d, F, cap["hq"][p], cap["hs"][p])
        assert np.array_equal(cap["down_sumi"][p], es), ("down", p, e)
        if spec.down_type != Q8_0:
            assert np.array_equal(cap["down_mins"][p], em), ("down", p, e)
    ref = L.moe_ffn(h, regime)
    assert rel_l2(out, ref) < TOL
    return int_slots


def test_headline_kernels_integers_bit_exact_extreme_ranges(ctx, orc):
    """One token, Mixtral shape (d 4096, FFN 14336, top-2, Q4_K): the tiled
    gate/up kernel and the split-K down kernel, on blocks with every byte 0xFF
    next to random ones and activations all +-127 (the largest |sumi| and
    |mins| the types allow)."""
    spec = LayerSpec(4, 2, 4096, 14336, Q4_K, seed=3, quantized=False)
    for parts in (spec.gate, spec.up, spec.down):
        for w in parts:
            plant_extremes(w, Q4_K)
    h = np.where(orc.normal(8, 4096) < 0, -3.0, 3.0).astype(np.float32).reshape(1, 4096)
    r = run_capture(ctx, orc, spec, 1, 0, h)
    assert np.abs(r[1]["xq"]).min() == 127
    assert check_ints(orc, spec, 1, 0, h, *r) == 2


def test_batch_kernels_integers_bit_exact_extreme_ranges(ctx, orc):
    """Decode batch on the int8 path (24 tokens over 4 experts, top-2): the
    streaming matrix-core kernel for experts with 5..32 rows, on blocks with
    every byte 0xFF next to random ones and activations all +-127."""
    spec = LayerSpec(4, 2, 1024, 2048, Q4_K, seed=5, quantized=False)
    for parts in (spec.gate, spec.up, spec.down):
        for w in parts:
            plant_extremes(w, Q4_K)
    h = np.where(orc.normal(9, 24 * 1024) < 0, -3.0, 3.0).astype(np.float32).reshape(24, 1024)
    r = run_capture(ctx, orc, spec, 24, 1, h)
    assert np.abs(r[1]["xq"]).min() == 127
    assert check_ints(orc, spec, 24, 1, h, *r) > 0


@pytest.mark.parametrize("d,ff,E,k,down_type,norm_topk,seed", [
    (2048, 768, 128, 8, Q4_K, True, 21),    # Qwen3-30B-A3B shape: register gate/up selecting 8 of 128, k_mv_down_exp<Q4_K>
    (2048, 1408, 64, 6, Q8_0, False, 22),   # DeepSeek-V2-Lite shape: 6 of 64, Q8_0 down over 44 blocks per row
    (2048, 1536, 32, 4, Q4_K, False, 23),   # moe-6b shape: 4 of 32, k_mv_down_exp<Q4_K> over 6 superblocks
])
def test_single_token_fine_grained_integers_bit_exact_extreme_ranges(ctx, orc, d, ff, E, k, down_type, norm_topk,
                                                                      seed):
    """One token through the fine-grained shapes' single-token kernels (the
    gate/up kernel over narrow rows that selects the experts itself, and the
    expert-ring down + combine), on blocks with every byte 0xFF next to random
    ones and activations all +-127: per-block integers of every selected
    expert's gate, up and down rows bit for bit against the oracle."""
    spec = LayerSpec(E, k, d, ff, Q4_K, seed=seed, quantized=False, down_type=down_type, norm_topk=norm_topk)
    for parts, t in ((spec.gate, Q4_K), (spec.up, Q4_K), (spec.down, down_type)):
        for w in parts:
            plant_extremes(w, t)
    h = np.where(orc.normal(seed, d) < 0, -3.0, 3.0).astype(np.float32).reshape(1, d)
    r = run_capture(ctx, orc, spec, 1, 0, h)
    assert np.abs(r[1]["xq"]).min() == 127
    assert check_ints(orc, spec, 1, 0, h, *r) == k


@pytest.mark.parametrize("S,regime,d,ff,E,k,types,seed", [
    (1, 0, 4096, 14336, 4, 2, (Q4_K, Q4_K), 1),   # tiled gate/up + split-K down, normal activations
    (1, 1, 4096, 8192, 8, 2, (Q4_K, Q6_K), 2),    # split-K down over tiled Q6_K rows
    (1, 0, 2048, 1408, 16, 6, (Q4_K, Q8_0), 3),   # register kernels (gate/up select, Q8_0 down + combine)
    (1, 0, 1024, 512, 8, 2, (Q8_0, Q8_0), 4),     # Q8_0 throughout
    (3, 0, 4096, 8192, 8, 2, (Q4_K, Q4_K), 5),    # few-rows kernels
    (8, 0, 4096, 8192, 4, 2, (Q4_K, Q4_K), 6),    # AVX2: f32 path for experts with >= 4 rows, few-rows for the rest
    (8, 1, 4096, 8192, 4, 2, (Q4_K, Q4_K), 7),    # few-rows up to 4 rows, matrix cores above
    (40, 1, 1024, 512, 4, 2, (Q4_K, Q4_K), 8),    # int8 matrix cores
    (12, 1, 1024, 768, 8, 2, (Q4_K, Q6_K), 9),    # matrix cores (gate/up), LDS-staged kernel (Q6_K down)
    (16, 1, 2048, 768, 128, 8, (Q4_K, Q4_K), 10),  # Qwen3 shape: narrow few-rows kernels for 1-3 rows
    (16, 0, 2048, 768, 128, 8, (Q4_K, Q4_K), 14),  # AVX2: f32 for experts with >= 4 rows, narrow few-rows for 1-3
    (6, 1, 2048, 1408, 64, 6, (Q4_K, Q8_0), 15),   # DeepSeek-V2-Lite shape: narrow few-rows kernels, Q8_0 down
    (24, 1, 1024, 768, 4, 2, (Q4_K, Q4_K), 12),   # streaming matrix-core kernel (<= 32 rows), 3 down superblocks
    (32, 1, 2048, 1536, 8, 2, (Q4_K, Q4_K), 13),  # few-rows kernels up to 4 rows, streaming kernel above
    (9, 1, 1024, 512, 8, 2, (Q8_0, Q8_0), 11),    # LDS-staged kernels, Q8_0
])
def test_moe_ffn_integers_bit_exact(ctx, orc, S, regime, d, ff, E, k, types, seed):
    spec = LayerSpec(E, k, d, ff, types[0], seed=seed, quantized=False, down_type=types[1])
    h = orc.normal(seed * 13 + S, S * d).reshape(S, d)
    r = run_capture(ctx, orc, spec, S, regime, h)
    assert check_ints(orc, spec, S, regime, h, *r) > 0


@pytest.mark.parametrize("S", [1, 3])
def test_moe_ffn_quantizes_exact_midpoints_half_away(ctx, orc, S):
    """The int8 rows of the layer input inside moe_ffn (the decode router's
    quantization for S < 4) round half away from zero (qdot.rs:361) on rows
    built from exact midpoints."""
    from tests.helpers import midpoint_rows, round_half_away

    spec = LayerSpec(8, 2, 4096, 8192, Q4_K, seed=20 + S, quantized=False)
    h, t = midpoint_rows(S, 4096, 256, seed=S)
    exp = round_half_away(t)
    assert (np.rint(t).astype(np.int8) != exp).any()
    r = run_capture(ctx, orc, spec, S, 0, h)
    assert np.array_equal(r[1]["xq"], exp)
    check_ints(orc, spec, S, 0, h, *r)
