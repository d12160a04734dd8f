"""Kernel-level parity of the HIP path against the oracle, through the C ABI.

Bar: bit-exact for integers (quantized activations, per-block integer
accumulators, routing indices, dispatch permutation); fp32 results within
1e-3 relative L2 of the oracle (the reference's AVX2 arithmetic).
"""
import numpy as np
import pytest

from tests.helpers import Q4_K, Q6_K, Q8_0, F32, random_blocks, rel_l2, row_bytes

pytestmark = pytest.mark.gpu

TOL = 1e-3  # fp32 relative L2 bound from the parity contract


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


@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 4096), (7, 14336), (2, 2048), (5, 768)])
def test_quantize_q8k_bit_exact(ctx, orc, rows, cols):
    x = orc.normal(rows * 31 + cols, rows * cols).reshape(rows, cols) * np.float32(3.0)
    x[0, :256] = 0.0  # zero block: scale 0, inv 0, q 0
    if cols >= 512:
        x[0, 300] = np.float32(1e30)  # huge value; the rest of the block quantizes to 0
    q, d, bs = ctx.quantize_q8k(dev(x))
    rq, rd, rbs = orc.q8k_quantize(x)
    assert np.array_equal(host(q), rq)
    assert np.array_equal(host(d).view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(host(bs), rbs)


@pytest.mark.parametrize("block,rows,cols", [(256, 1, 256), (256, 2, 4096), (256, 3, 14336), (32, 2, 1024),
                                              (32, 3, 96)])
def test_quantizers_round_half_away_at_exact_midpoints(ctx, orc, block, rows, cols):
    """qdot.rs:42 / :361 round half away from zero: blocks with amax =
    127 * 2^e put most elements on an exact midpoint (helpers.midpoint_rows),
    where a half-to-even rounding would give another value."""
    from tests.helpers import midpoint_rows, round_half_away

    x, t = midpoint_rows(rows, cols, block, seed=cols + rows)
    exp = round_half_away(t)
    assert (np.rint(t).astype(np.int8) != exp).any()
    if block == 256:
        q, d, s = ctx.quantize_q8k(dev(x))
        rq, rd, rs = orc.q8k_quantize(x)
    else:
        q, d, s = ctx.quantize_q8(dev(x))
        rq, rd, rs = orc.q8_quantize(x)
    assert np.array_equal(host(q), exp) and np.array_equal(rq, exp)
    assert np.array_equal(host(d).view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(host(s), rs)


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 1024), (2, 512), (4, 96)])
def test_quantize_q8_bit_exact(ctx, orc, rows, cols):
    x = orc.normal(rows * 17 + cols, rows * cols).reshape(rows, cols)
    x[-1, :32] = 0.0
    q, d, s16 = ctx.quantize_q8(dev(x))
    rq, rd, rs = orc.q8_quantize(x)
    assert np.array_equal(host(q), rq)
    assert np.array_equal(host(d).view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(host(s16), rs)


# S >= 8 runs the int8 matrix-core kernel (ragged row tiles, several 128-row token passes).
@pytest.mark.parametrize("rows,cols,S", [(64, 4096, 1), (37, 14336, 2), (16, 2048, 3), (9, 768, 1), (130, 4096, 3),
                                         (70, 4096, 8), (33, 768, 40), (130, 1024, 200), (64, 14336, 9)])
def test_q4k_block_sums_bit_exact(ctx, orc, rows, cols, S):
    w = random_blocks(Q4_K, rows, cols, seed=rows + cols)
    w[:: 144 * 5 + 7] = 0xFF  # every scale/min/nibble pattern, including the 6-bit high bits
    x = orc.normal(cols + S, S * cols).reshape(S, cols)
    q, d, bs = orc.q8k_quantize(x)
    sumi, mins = ctx.q4k_block_sums(dev(w), rows, cols, dev(q), dev(bs))
    sumi, mins = host(sumi), host(mins)
    rb = row_bytes(Q4_K, cols)
    for s in range(S):
        for r in range(rows):
            es, em = orc.q4k_block_acc(w[r * rb:(r + 1) * rb], cols, q[s], bs[s])
            assert np.array_equal(sumi[s, r], es), (s, r)
            assert np.array_equal(mins[s, r], em), (s, r)


@pytest.mark.parametrize("S", [1, 8, 33])
def test_q4k_block_sums_extreme_ranges(ctx, orc, S):
    """Largest integer magnitudes: every activation +-127 (16-sums +-2032), every
    6-bit scale and min 63, every nibble 15, next to all-zero superblocks."""
    rows, cols = 40, 1024
    w = np.full(rows * row_bytes(Q4_K, cols), 0xFF, np.uint8)
    w[: 144 * 3] = 0
    sign = np.where(orc.normal(5 + S, S * cols).reshape(S, cols) < 0, -1.0, 1.0).astype(np.float32)
    sign[:, 256:512] = 1.0  # a superblock of all +127
    sign[:, 512:768] = -1.0  # and one of all -127
    q, d, bs = orc.q8k_quantize(sign * 3.0)
    assert np.abs(q).min() == 127
    sumi, mins = ctx.q4k_block_sums(dev(w), rows, cols, dev(q), dev(bs))
    sumi, mins = host(sumi), host(mins)
    rb = row_bytes(Q4_K, cols)
    for s in range(S):
        for r in range(rows):
            es, em = orc.q4k_block_acc(w[r * rb:(r + 1) * rb], cols, q[s], bs[s])
            assert np.array_equal(sumi[s, r], es), (s, r)
            assert np.array_equal(mins[s, r], em), (s, r)


@pytest.mark.parametrize("rows,cols,S", [(40, 1024, 1), (33, 2048, 3), (9, 768, 2), (5, 14336, 1)])
def test_q6k_block_sums_bit_exact(ctx, orc, rows, cols, S):
    """Q6_K x Q8_K integers (avx2.rs:398-414): sumi = sum sc*q*x and offs =
    sum sc*bsum per superblock, on raw blocks (every 6-bit value, scales of
    both signs) and on quantized N(0, 0.02) rows."""
    x = orc.normal(rows + 7 * cols, S * cols).reshape(S, cols)
    q, d, bs = orc.q8k_quantize(x)
    rb = row_bytes(Q6_K, cols)
    raw = random_blocks(Q6_K, rows, cols, seed=rows * 5 + cols)
    quant = orc.quantize(Q6_K, orc.normal(rows * 3 + cols, rows * cols, 0.0, 0.02).reshape(rows, cols))
    for w in (raw, quant):
        sumi, offs = (host(t) for t in ctx.q6k_block_sums(dev(w), rows, cols, dev(q), dev(bs)))
        for s in range(S):
            for r in range(rows):
                es, eo = orc.q6k_block_acc(w[r * rb:(r + 1) * rb], cols, q[s], bs[s])
                assert np.array_equal(sumi[s, r], es), (s, r)
                assert np.array_equal(offs[s, r], eo), (s, r)


@pytest.mark.parametrize("rows,cols,S", [(40, 1024, 1), (33, 512, 3)])
def test_q8_0_block_sums_bit_exact(ctx, orc, rows, cols, S):
    w = random_blocks(Q8_0, rows, cols, seed=rows * 3 + cols)  # raw bytes include -128
    x = orc.normal(cols + 5 * S, S * cols).reshape(S, cols)
    q, d, s16 = orc.q8_quantize(x)
    p = host(ctx.q8_0_block_sums(dev(w), rows, cols, dev(q)))
    rb = row_bytes(Q8_0, cols)
    for s in range(S):
        for r in range(rows):
            assert np.array_equal(p[s, r], orc.q8_0_block_acc(w[r * rb:(r + 1) * rb], cols, q[s])), (s, r)


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 4096, 4096), (Q4_K, 14336, 4096), (Q4_K, 4096, 14336),
                                         (Q4_K, 1001, 3072), (Q4_K, 77, 8192), (Q4_K, 3, 12288), (Q4_K, 4099, 2048),
                                         (Q6_K, 4096, 4096), (Q6_K, 14336, 4096), (Q6_K, 4096, 14336),
                                         (Q6_K, 77, 768), (Q6_K, 1001, 3072),
                                         (Q8_0, 512, 1024), (Q8_0, 1024, 512)])
def test_matvec_decode_matches_oracle(ctx, orc, t, rows, cols):
    """Dense quantized matvec at decode batch 1 (the C2 shapes for Q4_K)."""
    w = random_blocks(t, rows, cols, seed=rows ^ cols)
    x = orc.normal(rows + cols, cols).reshape(1, cols)
    out = host(ctx.matmul(t, dev(w), rows, cols, dev(x)))
    ref = orc.matmul(t, w, rows, cols, x)
    assert rel_l2(out, ref) < TOL, rel_l2(out, ref)
    # and on the oracle's own Q8_K/Q8 bytes: same integers -> fp32 within a few ulp
    qf = orc.q8k_quantize if t in (Q4_K, Q6_K) else orc.q8_quantize
    q, d, s = qf(x)
    out2 = host(ctx.matvec_q8(t, dev(w), rows, cols, dev(q), dev(d), dev(s)))
    assert rel_l2(out2, ref) < 1e-5
    # the activation row's quantization is bit-exact wherever it runs (its own
    # kernel, or inside the Q4_K matvec for rows of at most 4096 columns), so
    # the whole call equals the matvec on the oracle's bytes bit for bit
    assert np.array_equal(out, out2)


@pytest.mark.parametrize("t", [Q4_K, Q8_0, Q6_K])
@pytest.mark.parametrize("S", [1, 2, 3, 4, 5, 8, 17])
@pytest.mark.parametrize("regime", [0, 1, 2])
def test_matmul_regimes_match_oracle(ctx, orc, t, S, regime):
    rows, cols = (192, 1024) if t in (Q4_K, Q6_K) else (160, 512)
    w = orc.quantize(t, orc.normal(S * 13 + t, rows * cols, 0.0, 0.02).reshape(rows, cols))
    x = orc.normal(S * 101 + regime, S * cols).reshape(S, cols)
    ctx.set_regime(regime)
    try:
        out = host(ctx.matmul(t, dev(w), rows, cols, dev(x)))
    finally:
        ctx.set_regime(0)
    ref = orc.matmul(t, w, rows, cols, x, regime)
    assert rel_l2(out, ref) < TOL, (S, regime, rel_l2(out, ref))


@pytest.mark.parametrize("t,rows,cols,S,regime", [(Q4_K, 2816, 2048, 128, 0), (Q4_K, 300, 2048, 40, 0),
                                                  (Q4_K, 192, 1024, 70, 0), (Q4_K, 64, 4096, 33, 2),
                                                  (Q4_K, 100, 512, 5, 0), (Q4_K, 77, 768, 2, 2),
                                                  (Q8_0, 2048, 1408, 128, 0), (Q8_0, 300, 1088, 40, 0),
                                                  (Q8_0, 64, 512, 5, 2), (Q8_0, 33, 4096, 20, 0)])
def test_matmul_f32_regime_plain_rows(ctx, orc, t, rows, cols, S, regime):
    """quant::matmul's f32 regime on GGUF rows: Q4_K through the bf16-split
    kernel (token blocks of 64, 32 and 16 rows, one and two K groups, ragged
    last blocks), Q8_0 through the fp32 GEMM (rows ending inside a 256-column
    span included): within a few fp32 roundings of the oracle's
    dequantize-and-multiply, and the same through an unaligned activation
    buffer (the fp32 GEMM)."""
    import torch

    w = random_blocks(t, rows, cols, seed=rows * 7 + cols)
    x = orc.normal(rows + S, S * cols).reshape(S, cols)
    ctx.set_regime(regime)
    try:
        out = host(ctx.matmul(t, dev(w), rows, cols, dev(x)))
        xb = torch.zeros(S * cols + 1, dtype=torch.float32, device="cuda")
        xb[1:].copy_(torch.from_numpy(x.ravel()))
        out_u = host(ctx.matmul(t, dev(w), rows, cols, xb[1:].view(S, cols)))
    finally:
        ctx.set_regime(0)
    ref = orc.matmul(t, w, rows, cols, x, regime)
    assert rel_l2(out, ref) < 3e-6, rel_l2(out, ref)
    assert rel_l2(out_u, ref) < 3e-6, rel_l2(out_u, ref)


@pytest.mark.parametrize("t,rows,cols,S,regime", [(Q4_K, 512, 4096, 1, 0), (Q4_K, 300, 2048, 5, 0),
                                                 (Q6_K, 64, 1024, 3, 0), (Q8_0, 100, 1024, 9, 1),
                                                 (Q4_K, 64, 1024, 12, 1), (F32, 8, 1024, 2, 0)])
def test_matmul_host_is_matmul(ctx, orc, t, rows, cols, S, regime):
    """kmoe_matmul_host, quant::matmul's own signature (quant.rs:229: host w,
    x and out): with host weights (copied for the call) and with resident
    device weights, the same bits as kmoe_matmul on device buffers."""
    w = (orc.normal(rows, rows * cols, 0.0, 0.02).view(np.uint8) if t == F32
         else random_blocks(t, rows, cols, seed=rows + cols))
    x = orc.normal(S + cols, S * cols).reshape(S, cols)
    ctx.set_regime(regime)
    try:
        ref = host(ctx.matmul(t, dev(w), rows, cols, dev(x)))
        a = ctx.matmul_host(t, w, rows, cols, x)
        b = ctx.matmul_host(t, dev(w), rows, cols, x)
    finally:
        ctx.set_regime(0)
    assert np.array_equal(a.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(b.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("E,d,S", [(8, 4096, 1), (8, 4096, 3), (8, 4096, 4), (8, 1024, 16), (128, 2048, 1),
                                   (128, 2048, 7), (64, 2048, 9), (50, 1024, 6), (8, 1000, 5), (8, 1000, 2),
                                   (8, 1004, 5), (8, 1004, 1),
                                   # batches: 3x4-kernel and dot_f32 orders side by side (48-row tile
                                   # remainders, S % 4 tokens, a last column chunk short of the staging width)
                                   (128, 2048, 270), (50, 1000, 297), (200, 1024, 330), (128, 2048, 512),
                                   (7, 512, 1031), (8, 1004, 400), (128, 2048, 70)])
def test_router_logits_bit_exact(ctx, orc, E, d, S):
    """F32 router matmul in the reference's summation order for this S."""
    wr = orc.normal(E * d, E * d, 0.0, 0.02).reshape(E, d)
    h = orc.normal(S * 7 + E, S * d).reshape(S, d)
    out = host(ctx.matmul(F32, dev(wr), E, d, dev(h)))
    ref = orc.matmul(F32, wr.view(np.uint8), E, d, h)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("E,k,d,S,norm,scale", [(8, 2, 4096, 1, True, 0.0), (8, 2, 1024, 16, True, 0.0),
                                                (128, 8, 2048, 33, True, 0.0), (64, 6, 2048, 5, False, 2.5),
                                                (60, 4, 1024, 3, True, 1.0)])
def test_route_matches_oracle(ctx, orc, E, k, d, S, norm, scale):
    wr = orc.normal(E + d, E * d, 0.0, 0.02).reshape(E, d)
    h = orc.normal(S + d, S * d).reshape(S, d)
    idx, w, logits = ctx.route(dev(wr), dev(h), k, norm, scale)
    from oracle.pyoracle import Layer

    L = Layer(E, k, d, 256, Q4_K, Q4_K, Q4_K, wr, [np.zeros(1, np.uint8)] * E, [np.zeros(1, np.uint8)] * E,
              [np.zeros(1, np.uint8)] * E, norm, scale)
    ridx, rw = L.route(h)
    assert np.array_equal(host(idx).astype(np.uint32), ridx)
    # p = expf(v - m): the device uses a correctly rounded expf, glibc's is
    # within 0.502 ulp, so weights agree to a few ulp.
    assert np.allclose(host(w), rw, rtol=1e-6, atol=0)


@pytest.mark.parametrize("E,k,S", [(8, 2, 1), (8, 2, 3), (8, 2, 5), (128, 8, 1), (128, 8, 6), (64, 6, 2)])
def test_route_nan_logit_selects_in_index_order(ctx, orc, E, k, S):
    """A NaN in router row E/2 makes that logit NaN for every token; the
    reference's softmax then makes every p NaN and its comparator falls back
    to index order (transformer.rs:479-484): experts 0..k-1, NaN weights. S < 4
    runs the fused decode router, S >= 4 the logits + top-k kernels."""
    d = 1024
    wr = orc.normal(E + 3, E * d, 0.0, 0.02).reshape(E, d)
    wr[E // 2, 5] = np.nan
    h = orc.normal(S + 11, S * d).reshape(S, d)
    idx, w, logits = ctx.route(dev(wr), dev(h), k, True, 0.0)
    from oracle.pyoracle import Layer

    z = [np.zeros(1, np.uint8)] * E
    ridx, rw = Layer(E, k, d, 256, Q4_K, Q4_K, Q4_K, wr, z, z, z, True, 0.0).route(h)
    assert ridx.tolist() == [list(range(k))] * S
    assert np.array_equal(host(idx).astype(np.uint32), ridx)
    assert np.isnan(host(w)).all() and np.isnan(rw).all()


@pytest.mark.parametrize("S,k,E", [(1, 2, 8), (16, 2, 8), (7, 6, 64), (512, 2, 8), (700, 8, 128), (2048, 8, 128),
                                   (3, 1, 1), (100, 4, 512)])
def test_dispatch_bit_exact(ctx, orc, S, k, E):
    rng = np.random.default_rng(S * 31 + E)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(S)]).astype(np.uint32)
    perm, off = ctx.dispatch(dev(idx.view(np.int32)), E)
    rp, ro = orc.dispatch(idx, E)
    assert np.array_equal(host(perm).view(np.uint32), rp)
    assert np.array_equal(host(off).view(np.uint32), ro)


def test_dispatch_all_to_one_expert(ctx, orc):
    idx = np.zeros((3000, 1), np.uint32)
    perm, off = ctx.dispatch(dev(idx.view(np.int32)), 4)
    assert np.array_equal(host(perm).view(np.uint32), np.arange(3000, dtype=np.uint32))
    assert host(off).tolist() == [0, 3000, 3000, 3000, 3000]


# ------------------------------------------------- the other quant::matmul types
_XT = {"Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q5_K": 13, "F16": 1, "BF16": 30}


def _xt_weights(orc, t, rows, cols, seed):
    """qdot.rs:275-299's generator (xorshift32 bytes, the f16 scale and min
    fields set to 0.002); F16 / BF16 rows of N(0, 0.02)."""
    if t in (1, 30):
        v = orc.normal(seed, rows * cols, 0.0, 0.02)
        return v.astype(np.float16).view(np.uint8) if t == 1 else (v.view(np.uint32) >> 16).astype(np.uint16).view(
            np.uint8)
    w = orc.xorshift_bytes(seed, orc.bytes_for(t, rows * cols)).copy()
    blk = w.reshape(-1, orc.type_size(t))
    h = orc.f16_bits(0.002)
    for o in {2: [0], 6: [0], 3: [0, 2], 7: [0, 2], 13: [0, 2]}[t]:
        blk[:, o] = h & 0xFF
        blk[:, o + 1] = h >> 8
    return w


@pytest.mark.parametrize("name", list(_XT))
@pytest.mark.parametrize("regime", [0, 1, 2])
def test_matmul_other_types_bit_exact(ctx, orc, name, regime):
    """quant::matmul over F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1 and Q5_K weights:
    the reference's bits in every regime and row count (dequantize + the f32
    orders; the AVX2 dot of the unpacked rows with Q8 activations)."""
    t = _XT[name]
    rows, cols = 96, 1024
    w = _xt_weights(orc, t, rows, cols, 17 + t)
    ctx.set_regime(regime)
    try:
        for S in (1, 3, 5, 17):
            x = orc.normal(40 + S + t, S * cols).reshape(S, cols)
            out = host(ctx.matmul(t, dev(w), rows, cols, dev(x)))
            ref = orc.matmul(t, w, rows, cols, x, regime)
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (name, regime, S)
    finally:
        ctx.set_regime(0)


def test_matmul_other_types_odd_widths_and_host_seam(ctx, orc):
    """F16 rows of 1000 columns (not a multiple of 8: quant::dot order at
    every S) and Q5_K through the host-slice entry point."""
    w = _xt_weights(orc, 1, 40, 1000, 5)
    for S in (2, 6):
        x = orc.normal(50 + S, S * 1000).reshape(S, 1000)
        out = host(ctx.matmul(1, dev(w), 40, 1000, dev(x)))
        assert np.array_equal(out.view(np.uint32), orc.matmul(1, w, 40, 1000, x).view(np.uint32))
    w = _xt_weights(orc, 13, 64, 512, 6)
    x = orc.normal(61, 2 * 512).reshape(2, 512)
    a = ctx.matmul_host(13, w, 64, 512, x)
    assert np.array_equal(a.view(np.uint32), orc.matmul(13, w, 64, 512, x).view(np.uint32))
