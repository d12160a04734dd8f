"""Pins the CPU oracle before anything is compared against it.

Each test replays one of the reference's own unit tests (same generators,
same sizes, same tolerances; file:line cited), or checks the oracle against
something the mathematics fixes: brute-force integer sums, float64 dequantized
products, a stable sort, an argsort of the logits. None of them retypes the
oracle's formula.
"""
import numpy as np
import pytest

from oracle.pyoracle import (BF16, F16, F32, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, REGIME_AVX2,
                              REGIME_EXACT, REGIME_INT8)


def _blocks(orc, t, n, seed, scale):
    """qdot.rs:275-299 / avx2.rs:198-208: xorshift32 bytes, f16 scales overwritten."""
    w = orc.xorshift_bytes(seed, orc.bytes_for(t, n)).copy()
    bs = orc.type_size(t)
    offs = {Q8_0: [0], Q4_0: [0], Q5_0: [0], Q4_1: [0, 2], Q5_1: [0, 2], Q4_K: [0, 2], Q5_K: [0, 2],
            Q6_K: [208]}[t]
    h = orc.f16_bits(scale)
    blk = w.reshape(-1, bs)
    for o in offs:
        blk[:, o] = h & 0xFF
        blk[:, o + 1] = h >> 8
    return w


def test_q8_0_and_q4_0_known_values(orc):
    # quant.rs:375-394
    b = np.zeros(34, np.uint8)
    h = orc.f16_bits(0.5)
    b[0], b[1] = h & 0xFF, h >> 8
    b[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    y = orc.dequant(Q8_0, b, 32)
    assert y[0] == -8.0 and y[31] == 7.5
    b = np.zeros(18, np.uint8)
    h = orc.f16_bits(2.0)
    b[0], b[1] = h & 0xFF, h >> 8
    b[2] = 0x9F
    y = orc.dequant(Q4_0, b, 32)
    assert y[0] == 14.0 and y[16] == 2.0 and y[1] == -16.0


def test_q6_k_known_values(orc):
    """quant.rs:180-201 on a hand-built block: element e = 128h + 32r + l takes
    the low (r < 2) or high nibble of ql[64h + 32(r&1) + l], bits 2r..2r+1 of
    qh[32h + l] as bits 4-5, and the signed scale sc[e/16]; y = d*sc*(q - 32)."""
    b = np.zeros(210, np.uint8)
    h = orc.f16_bits(0.5)
    b[208], b[209] = h & 0xFF, h >> 8
    b[192:208] = 2
    b[192 + 5] = np.uint8(253)  # sc[5] = -3
    b[0] = 0x0F                 # e=0: low nibble 15
    b[128] = 0x03               # e=0: qh bits 0-1 = 3 -> q = 63
    b[16] = 0x50                # e=80 (h=0, r=2, l=16): high nibble 5
    b[128 + 16] = 0x10          # e=80: qh bits 4-5 = 1 -> q = 21
    b[97] = 0x07                # e=161 (h=1, r=1, l=1): low nibble of ql[64+32+1]
    b[128 + 33] = 0x08          # e=161: qh bits 2-3 = 2 -> q = 39
    y = orc.dequant(Q6_K, b, 256)
    assert y[0] == 0.5 * 2 * 31
    assert y[80] == 0.5 * -3 * (21 - 32)
    assert y[161] == 0.5 * 2 * (39 - 32)
    assert y[64] == 0.5 * 2 * -32 and y[255] == 0.5 * 2 * -32
    assert y[81] == 0.5 * -3 * -32  # rest of sub-block 5: q = 0


def test_known_bpw(orc):
    # kestrel-gguf types.rs:300-307
    for t, bpw in [(Q4_0, 4.5), (Q8_0, 8.5), (Q4_K, 4.5), (Q6_K, 6.5625)]:
        assert orc.type_size(t) * 8 / orc.block_size(t) == bpw
    assert orc.bytes_for(Q4_K, 512) == 288
    assert orc.bytes_for(Q4_K, 100) is None
    # Row bytes of the shapes this build runs (types.rs:184-191).
    assert orc.bytes_for(Q4_K, 4096) == 2304 and orc.bytes_for(Q4_K, 14336) == 8064
    assert orc.bytes_for(Q8_0, 1024) == 1088 and orc.bytes_for(Q8_0, 512) == 544


def test_f16_conversion_is_exact(orc):
    # half 2.7.1 to_f32 is the IEEE conversion: check every finite f16 against numpy.
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    lib = orc.lib()
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits[::97]], np.float32)
    r = ref[::97]
    fin = np.isfinite(r)
    assert np.array_equal(got[fin].view(np.uint32), r[fin].view(np.uint32))
    # f32 -> f16 round-to-nearest-even agrees with numpy on random values.
    v = orc.normal(5, 4000, 0.0, 3.0) * np.float32(10.0) ** orc.normal(6, 4000, 0.0, 2.0).clip(-6, 3.5)
    mine = np.array([orc.f16_bits(float(x)) for x in v], np.uint16)
    assert np.array_equal(mine, v.astype(np.float16).view(np.uint16))


def test_matmul_matches_naive(orc):
    # quant.rs:397-411 (F32, S=3 < 4: dequant + quant::dot)
    rows, cols, s = 37, 64, 3
    i = np.arange(rows * cols)
    wf = (((i * 31) % 17).astype(np.float32) - 8.0) * np.float32(0.1)
    x = ((np.arange(s * cols) % 5).astype(np.float32) - 2.0)
    out = orc.matmul(F32, wf.view(np.uint8), rows, cols, x.reshape(s, cols))
    e = x.reshape(s, cols).astype(np.float64) @ wf.reshape(rows, cols).astype(np.float64).T
    assert np.abs(out - e).max() < 1e-3


def _f16le(v):
    return np.array([v], np.float16).view(np.uint8)


def test_q4_1_q5_0_q5_1_known_values(orc):
    """Hand-built 32-blocks; element j (< 16) is the low nibble of qs[j], element
    j + 16 its high nibble; Q5 types take bit j of the 32-bit qh word as bit 4
    of element j (ggml's block_q5_0 / block_q5_1)."""
    j = np.arange(16)
    qs = (j | ((15 - j) << 4)).astype(np.uint8)
    nib = np.concatenate([j, 15 - j]).astype(np.float64)
    # Q4_1: d = 0.5, m = -1.0 -> q * d + m
    b = np.concatenate([_f16le(0.5), _f16le(-1.0), qs])
    assert np.array_equal(orc.dequant(Q4_1, b, 32), (nib * 0.5 - 1.0).astype(np.float32))
    qh = 0b1010_0101_1100_0011_0000_1111_1001_0110
    hbit = np.array([(qh >> i) & 1 for i in range(32)], np.float64)
    qhb = np.array([qh], np.uint32).view(np.uint8)
    # Q5_0: d = 0.25 -> ((nibble | bit << 4) - 16) * d
    b = np.concatenate([_f16le(0.25), qhb, qs])
    assert np.array_equal(orc.dequant(Q5_0, b, 32), ((nib + 16 * hbit - 16) * 0.25).astype(np.float32))
    # Q5_1: d = 0.125, m = 2.0 -> (nibble | bit << 4) * d + m
    b = np.concatenate([_f16le(0.125), _f16le(2.0), qhb, qs])
    assert np.array_equal(orc.dequant(Q5_1, b, 32), ((nib + 16 * hbit) * 0.125 + 2.0).astype(np.float32))


def test_q5_k_known_values(orc):
    """Hand-built Q5_K superblock (ggml's block_q5_K: d, dmin, 12 scale bytes,
    qh[32], qs[128]). Sub-blocks 2k and 2k+1 take the low and high nibbles of
    qs[32k + l] and bits 2k and 2k+1 of qh[l]; sub-block j has scale 2j+1
    and min j, packed into the 12 scale bytes as scale_min_k4 reads them
    (quant.rs:54-61)."""
    d, dmin = 0.5, 0.25
    sc = np.array([1, 3, 5, 7, 9, 11, 13, 15], np.uint8)  # sub-block j: scale j*2+1 (sub-blocks 0..7)
    mn = np.array([0, 1, 2, 3, 4, 5, 6, 7], np.uint8)
    scales = np.zeros(12, np.uint8)
    scales[0:4] = sc[0:4]  # j < 4: scale = q[j] & 63, min = q[j + 4] & 63
    scales[4:8] = mn[0:4]
    scales[8:12] = (sc[4:8] & 0xF) | ((mn[4:8] & 0xF) << 4)  # j >= 4: low 4 bits in q[j + 4]
    scales[0:4] |= (sc[4:8] >> 4) << 6  # high 2 bits in the top bits of q[j - 4] / q[j]
    scales[4:8] |= (mn[4:8] >> 4) << 6
    l = np.arange(32)
    qs = np.concatenate([((l + k) & 0xF) | (((31 - l - k) & 0xF) << 4) for k in range(4)]).astype(np.uint8)
    qh = ((l * 37 + 11) & 0xFF).astype(np.uint8)
    b = np.concatenate([_f16le(d), _f16le(dmin), scales, qh, qs])
    assert b.size == 176
    exp = np.empty(256)
    for k in range(4):
        for half, s in ((0, 2 * k), (1, 2 * k + 1)):
            nib = ((l + k) & 0xF) if half == 0 else ((31 - l - k) & 0xF)
            hi = (qh >> s) & 1
            exp[64 * k + 32 * half + l] = (d * sc[s]) * (nib + 16 * hi) - dmin * mn[s]
    got = orc.dequant(Q5_K, b, 256)
    assert np.allclose(got, exp.astype(np.float32), rtol=0, atol=1e-6)
    q, usc, umn = orc.unpack(Q5_K, b, 256)
    assert q.min() >= 0 and q.max() <= 31


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K])
def test_unpack_matches_dequantization_exactly(orc, t):
    # qdot.rs:301-315
    n = 1024
    w = _blocks(orc, t, n, 7, 0.01)
    wf = orc.dequant(t, w, n)
    q, sc, mn = orc.unpack(t, w, n)
    i = np.arange(n)
    v = sc[i // 16] * q.astype(np.float32) - mn[i // 16]
    assert np.all(np.abs(v - wf) <= 1e-5 * np.maximum(np.abs(wf), 1.0))


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K, Q5_1, Q4_1, Q5_0, Q5_K])
def test_dot_close_to_float(orc, t):
    # qdot.rs:317-333
    n = 1024
    i = np.arange(n)
    x = (((i * 37) % 101).astype(np.float32) - 50.0) / np.float32(25.0)
    q, d, s16 = orc.q8_quantize(x)
    w = _blocks(orc, t, n, 3, 0.01)
    wf = orc.dequant(t, w, n)
    exact = orc.lib().orc_quant_dot(wf.ctypes.data, x.ctypes.data, n)
    uq, usc, umn = orc.unpack(t, w, n)
    fast = orc.lib().orc_dot_unpacked_avx2(uq.ctypes.data, usc.ctypes.data, umn.ctypes.data, n, q.ctypes.data,
                                           d.ctypes.data, s16.ctypes.data)
    tol = float(np.abs(wf).sum()) * 2.0 / 127.0 * 0.6
    assert abs(exact - fast) <= max(tol, 1e-3)


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K])
def test_fused_kernels_match_unpacked_reference(orc, t):
    # avx2.rs:184-223
    n = 2048
    i = np.arange(n)
    x = (((i * 53) % 211).astype(np.float32) - 105.0) / np.float32(40.0)
    q, d, s16 = orc.q8_quantize(x)
    q, d, s16 = q[0], d[0], s16[0]
    w = _blocks(orc, t, n, 9, 0.02)
    uq, usc, umn = orc.unpack(t, w, n)
    r = np.float32(0.0)
    for k in range(n // 16):  # scalar reference over the unpacked representation
        p = int(np.dot(uq[16 * k:16 * k + 16].astype(np.int32), q[16 * k:16 * k + 16].astype(np.int32)))
        r = np.float32(r + d[k // 2] * (usc[k] * np.float32(p) - umn[k] * np.float32(s16[k])))
    L = orc.lib()
    f = {Q8_0: lambda: L.orc_dot_q8_0(w.ctypes.data, n, q.ctypes.data, d.ctypes.data),
         Q4_0: lambda: L.orc_dot_q4_0(w.ctypes.data, n, q.ctypes.data, d.ctypes.data),
         Q4_K: lambda: L.orc_dot_q4_k(w.ctypes.data, n, q.ctypes.data, d.ctypes.data, s16.ctypes.data)}[t]
    fused = f()
    generic = L.orc_dot_unpacked_avx2(uq.ctypes.data, usc.ctypes.data, umn.ctypes.data, n, q.ctypes.data,
                                      d.ctypes.data, s16.ctypes.data)
    tol = 1e-4 * max(abs(float(r)), 1.0)
    assert abs(fused - r) <= tol
    assert abs(generic - r) <= tol


def test_gemm_matches_naive(orc):
    # avx2.rs:312-330
    for rows, s_rows, cols in [(7, 9, 64), (3, 4, 8), (1, 1, 24), (10, 3, 256)]:
        w = (((np.arange(rows * cols) * 7) % 13).astype(np.float32) - 6.0) * np.float32(0.1)
        x = (((np.arange(s_rows * cols) * 5) % 11).astype(np.float32) - 5.0) * np.float32(0.2)
        res = np.empty(rows * s_rows, np.float32)
        orc.lib().orc_gemm_f32(w.ctypes.data, rows, x.ctypes.data, s_rows, cols, res.ctypes.data)
        e = w.reshape(rows, cols).astype(np.float64) @ x.reshape(s_rows, cols).astype(np.float64).T
        assert np.abs(res.reshape(rows, s_rows) - e).max() < 1e-3


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_q8k_kernels_match_dequantized_math(orc, t):
    # avx2.rs:425-460 (both Q8_K kernels, same inputs and tolerance)
    n = 2048
    i = np.arange(n)
    x = (((i * 53) % 211).astype(np.float32) - 105.0) / np.float32(40.0)
    q, d, bs = orc.q8k_quantize(x)
    w = _blocks(orc, t, n, 7, 0.02)
    uq, usc, umn = orc.unpack(t, w, n)
    wv = (usc[i // 16] * uq.astype(np.float32) - umn[i // 16]).astype(np.float64)
    r = float(np.sum(wv * q[0].astype(np.float64) * d[0][i // 256].astype(np.float64)))
    f = orc.lib().orc_dot_q4_k_8k if t == Q4_K else orc.lib().orc_dot_q6_k_8k
    got = f(w.ctypes.data, n, q.ctypes.data, d.ctypes.data, bs.ctypes.data)
    assert abs(got - r) <= 1e-3 * max(abs(r), 1.0)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_q4k_block_accumulators_match_bruteforce(orc, seed):
    n = 4096
    x = orc.normal(seed, n)
    q, d, bs = orc.q8k_quantize(x)
    w = orc.quantize(Q4_K, orc.normal(seed + 100, n, 0.0, 0.02).reshape(1, n))
    wr = orc.xorshift_bytes(seed, w.size)  # raw bytes: every scale/min/nibble pattern
    for ww in (w, wr):
        s, m = orc.q4k_block_acc(ww, n, q[0], bs[0])
        s2, m2 = orc.q4k_block_acc_bruteforce(ww, n, q[0], bs[0])
        assert np.array_equal(s.astype(np.int64), s2) and np.array_equal(m.astype(np.int64), m2)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_q6k_block_accumulators_match_bruteforce(orc, seed):
    n = 4096
    x = orc.normal(seed, n)
    q, d, bs = orc.q8k_quantize(x)
    w = orc.quantize(Q6_K, orc.normal(seed + 100, n, 0.0, 0.02).reshape(1, n))
    wr = orc.xorshift_bytes(seed, w.size)  # raw bytes: every 6-bit value and signed scale
    for ww in (w, wr):
        s, o = orc.q6k_block_acc(ww, n, q[0], bs[0])
        s2, o2 = orc.q6k_block_acc_bruteforce(ww, n, q[0])
        assert np.array_equal(s.astype(np.int64), s2) and np.array_equal(o.astype(np.int64), o2)


def test_q8_0_block_accumulators_match_bruteforce(orc):
    n = 1024
    q, d, s16 = orc.q8_quantize(orc.normal(4, n))
    w = orc.xorshift_bytes(11, orc.bytes_for(Q8_0, n))  # includes -128 weights
    p = orc.q8_0_block_acc(w, n, q[0])
    wq = w.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64)
    ref = (wq * q[0].reshape(-1, 32).astype(np.int64)).sum(1)
    assert np.array_equal(p.astype(np.int64), ref)


@pytest.mark.parametrize("block", [256, 32])
def test_q8_quantizers_round_half_away_at_exact_midpoints(orc, block):
    """qdot.rs:42 / :361: `(xs[j] * inv).round() as i32` rounds half away from
    zero. Blocks with amax = 127 * 2^e make scale and x * inv exact, so most
    elements sit on a midpoint: a half-to-even rounding (rint) fails here."""
    from tests.helpers import midpoint_rows, round_half_away

    x, t = midpoint_rows(4, 2048, block, seed=block)
    exp = round_half_away(t)
    assert (np.rint(t).astype(np.int8) != exp).sum() > 500  # the inputs tell the two rules apart
    q, d, s = (orc.q8k_quantize if block == 256 else orc.q8_quantize)(x)
    assert np.array_equal(q, exp)
    scale = np.abs(x.reshape(4, -1, block)).max(2) / np.float32(127.0)
    assert np.array_equal(d, scale.astype(np.float32)) and np.all(np.log2(d) == np.round(np.log2(d)))
    assert np.array_equal(s, exp.reshape(4, -1, 16).astype(np.int32).sum(2))


def test_q8k_quantize_semantics(orc):
    # qdot.rs:347-367: scale = amax/127, q = round(x / scale) clamped; bsums per 16.
    x = orc.normal(9, 1024)
    x[:256] = 0.0  # zero block -> scale 0, q 0
    q, d, bs = orc.q8k_quantize(x)
    assert d[0, 0] == 0.0 and not q[0, :256].any()
    ax = np.abs(x.reshape(-1, 256)).max(1)
    assert np.array_equal(d[0], (ax / np.float32(127.0)).astype(np.float32))
    recon = q[0].astype(np.float64) * np.repeat(d[0], 256)
    assert np.all(np.abs(recon - x) <= np.repeat(d[0], 256) * 0.5 + 1e-12)
    assert np.array_equal(bs[0], q[0].reshape(-1, 16).astype(np.int32).sum(1))


@pytest.mark.parametrize("t,n", [(Q8_0, 1024), (Q4_K, 4096), (Q6_K, 4096)])
def test_quantizers_round_trip(orc, t, n):
    x = orc.normal(12, n, 0.0, 0.02)
    w = orc.quantize(t, x.reshape(1, n))
    y = orc.dequant(t, w, n)
    if t == Q8_0:  # |x - y| <= d/2 + |q| * (f16 rounding of d), d = amax/127
        amax = np.abs(x.reshape(-1, 32)).max(1)
        bound = np.repeat(amax / 127.0, 32) * (0.5 + 127 * 2.0 ** -11) + 1e-7
    elif t == Q4_K:  # per sub-block range / 15 / 2 plus the 6-bit rounding of scale and min
        r = x.reshape(-1, 32)
        bound = np.repeat((r.max(1) - np.minimum(r.min(1), 0)) / 15.0, 32) * 1.5 + 1e-4
    else:  # step ~ amax_16/32 per 16-block (+ the 8-bit rounding of the scale); +amax clamps to 31 steps
        r = x.reshape(-1, 16)
        step = np.abs(r).max(1) / 32.0
        d = np.repeat(step.reshape(-1, 16).max(1) / 127.0, 16)
        bound = np.repeat(step + d, 16) * 1.5 + 1e-7
    assert np.all(np.abs(x - y) <= bound)
    tol = {Q8_0: 0.01, Q4_K: 0.12, Q6_K: 0.05}[t]
    assert np.sqrt(np.mean((x - y) ** 2)) / np.sqrt(np.mean(x ** 2)) < tol


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q4_0, Q4_1, Q5_0, Q5_1, Q5_K, F16, BF16])
def test_matmul_regimes(orc, t):
    """quant.rs:242/262/282/311: S>=4 is f32-exact; S<4 carries the int8
    activations' error (Q8_K or Q8 rows), except F16/BF16 weights, which take
    dequantize + quant::dot at every S."""
    rows, cols = 64, 1024
    rb = orc.bytes_for(t, cols)
    if t in (F16, BF16):
        wf32 = orc.normal(21, rows * cols, 0.0, 0.02)
        w = wf32.astype(np.float16).view(np.uint8) if t == F16 else \
            (wf32.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    elif t in (Q4_K, Q6_K):
        w = orc.quantize(t, orc.normal(21, rows * cols, 0.0, 0.02).reshape(rows, cols))
    else:
        w = _blocks(orc, t, rows * cols, 21, 0.002)
    wf = np.stack([orc.dequant(t, w[r * rb:(r + 1) * rb], cols) for r in range(rows)]).astype(np.float64)
    for S in (1, 3, 4, 7):
        x = orc.normal(30 + S, S * cols).reshape(S, cols)
        e = x.astype(np.float64) @ wf.T
        for regime in (REGIME_AVX2, REGIME_INT8, REGIME_EXACT):
            out = orc.matmul(t, w, rows, cols, x, regime)
            rel = np.linalg.norm(out - e) / np.linalg.norm(e)
            exact = (regime == REGIME_EXACT) or (regime == REGIME_AVX2 and S >= 4) or t in (F16, BF16)
            assert rel < (1e-6 if exact else 2e-2), (S, regime, rel)


def test_route_matches_argsort_of_logits(orc):
    """transformer.rs:472-496 against a float64 softmax + argsort (distinct logits)."""
    rng = np.random.default_rng(0)
    for E, k, norm in [(8, 2, True), (128, 8, True), (64, 6, False)]:
        logits = rng.standard_normal((50, E)).astype(np.float32) * 3
        idx, w = orc.route_from_logits(logits, k, norm, 0.0)
        l64 = logits.astype(np.float64)
        p = np.exp(l64 - l64.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        ref_idx = np.argsort(-l64, axis=1, kind="stable")[:, :k]
        assert np.array_equal(idx, ref_idx)
        ref_w = np.take_along_axis(p, ref_idx, 1)
        if norm:
            ref_w = ref_w / ref_w.sum(1, keepdims=True)
        assert np.allclose(w, ref_w, rtol=2e-6, atol=0)
    # weights_scale multiplies (MoeInfo.weights_scale, 0 or 1 = none)
    i1, w1 = orc.route_from_logits(logits[:4], 6, False, 2.5)
    i0, w0 = orc.route_from_logits(logits[:4], 6, False, 1.0)
    assert np.array_equal(i0, i1) and np.array_equal(w1, (w0 * np.float32(2.5)).astype(np.float32))


def test_route_ties_prefer_lower_index(orc):
    logits = np.zeros((2, 8), np.float32)
    logits[1, [6, 2, 5]] = 1.0
    idx, w = orc.route_from_logits(logits, 3, True, 0.0)
    assert idx[0].tolist() == [0, 1, 2] and idx[1].tolist() == [2, 5, 6]
    assert np.allclose(w, 1.0 / 3.0)


def test_route_nan_and_inf_logits_fall_back_to_index_order(orc):
    """transformer.rs:479-484. A NaN logit leaves m = the max of the others
    (f32::max skips NaN), so its p and then `sum` are NaN and every p /= sum
    is NaN; a +inf logit gives exp(inf - inf) = NaN the same way. The sort's
    comparator maps NaN to Equal and falls back to ascending index, so such a
    row selects experts 0..k-1 with NaN weights (the 2^-14 floor's f32::max
    also skips NaN). A -inf logit is just p = 0."""
    E, k = 16, 4
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((4, E)).astype(np.float32)
    logits[0, 7] = np.nan
    logits[1, 3] = np.inf
    logits[2, :] = np.nan
    logits[3, 0] = -np.inf
    idx, w = orc.route_from_logits(logits, k, True, 0.0)
    assert idx[:3].tolist() == [[0, 1, 2, 3]] * 3 and np.isnan(w[:3]).all()
    ref = np.argsort(-logits[3].astype(np.float64), kind="stable")[:k]
    assert idx[3].tolist() == ref.tolist() and 0 not in ref and np.isfinite(w[3]).all()


def test_dispatch_is_stable_sort(orc):
    rng = np.random.default_rng(3)
    for S, k, E in [(1, 2, 8), (16, 2, 8), (512, 8, 128), (7, 6, 64)]:
        idx = np.stack([rng.choice(E, k, replace=False) for _ in range(S)]).astype(np.uint32)
        perm, off = orc.dispatch(idx, E)
        assert np.array_equal(perm, np.argsort(idx.reshape(-1), kind="stable"))
        assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(idx.reshape(-1), minlength=E))]))


def _small_layer(orc, t, E=4, k=2, d=256, ff=256, seed=0):
    rng_seed = seed * 1000
    router = orc.normal(rng_seed + 1, E * d, 0.0, 0.02).reshape(E, d)
    mk = lambda s, r, c: orc.quantize(t, orc.normal(s, r * c, 0.0, 0.02).reshape(r, c))
    gate = [mk(rng_seed + 10 + e, ff, d) for e in range(E)]
    up = [mk(rng_seed + 20 + e, ff, d) for e in range(E)]
    down = [mk(rng_seed + 30 + e, d, ff) for e in range(E)]
    return orc.Layer(E, k, d, ff, t, t, t, router, gate, up, down)


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
def test_moe_ffn_matches_float64_layer(orc, t):
    """transformer.rs:513-570 against a float64 evaluation of the same layer."""
    L = _small_layer(orc, t)
    d, ff, E, k = L.d, L.ff, L.n_expert, L.k
    rb_d, rb_f = orc.bytes_for(t, d), orc.bytes_for(t, ff)
    deq = lambda w, r, c, rb: np.stack([orc.dequant(t, w[i * rb:(i + 1) * rb], c) for i in range(r)]).astype(np.float64)
    G = [deq(L.gate[e], ff, d, rb_d) for e in range(E)]
    U = [deq(L.up[e], ff, d, rb_d) for e in range(E)]
    D = [deq(L.down[e], d, ff, rb_f) for e in range(E)]
    for S in (1, 5, 12):
        h = orc.normal(77 + S, S * d).reshape(S, d)
        idx, w = L.route(h)
        ref = np.zeros((S, d))
        for s in range(S):
            for j in range(k):
                e = idx[s, j]
                g = G[e] @ h[s].astype(np.float64)
                u = U[e] @ h[s].astype(np.float64)
                a = g / (1 + np.exp(-g)) * u
                ref[s] += w[s, j] * (D[e] @ a)
        for regime in (REGIME_AVX2, REGIME_EXACT, REGIME_INT8):
            out = L.moe_ffn(h, regime)
            rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
            assert rel < (3e-2 if regime == REGIME_INT8 else 2e-2), (S, regime, rel)
        # AVX2 with S=12: experts with >=4 rows are f32-exact, the rest carry Q8 error.
        out = L.moe_ffn(h, REGIME_EXACT)
        assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-5


def test_matmul_thread_count_independent(orc):
    rows, cols = 200, 512
    w = orc.quantize(Q4_K, orc.normal(5, rows * cols, 0, 0.02).reshape(rows, cols))
    x = orc.normal(6, 2 * cols).reshape(2, cols)
    a = orc.matmul(Q4_K, w, rows, cols, x, threads=1)
    b = orc.matmul(Q4_K, w, rows, cols, x, threads=0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_bench_gemv_runs(orc):
    # quant.rs:348-368 (small sizes here; the full metric runs in bench.py)
    assert orc.bench_gemv(Q4_K, 256, 4096, 2, 1) > 0


# ------------------------------------------------------------- shared expert
def _shared_case(orc, S, t, seed):
    from tests.helpers import LayerSpec

    d, ff = 1024, 768 if t == Q4_K else 512
    spec = LayerSpec(1, 1, d, ff, t, seed=seed)
    h = orc.normal(seed + 5, S * d).reshape(S, d)
    return spec, h, d, ff


@pytest.mark.parametrize("S", [1, 3, 4, 9])
@pytest.mark.parametrize("regime", [0, 1, 2])
def test_shared_expert_equals_single_expert_layer(orc, S, regime):
    """With no gate vector the shared expert adds exactly what a 1-expert, top-1
    layer with the same tensors computes: routing gives weight exp(0)/1 = 1 to
    every row and its matmul runs over the same S rows (same regime)."""
    for t in (Q8_0, Q4_K):
        spec, h, d, ff = _shared_case(orc, S, t, seed=S + 10 * regime)
        ref = spec.oracle_layer().moe_ffn(h, regime)
        got = orc.shared_expert_add(np.zeros((S, d), np.float32), h, d, ff, (t, t, t), spec.gate[0], spec.up[0],
                                    spec.down[0], None, regime)
        assert np.array_equal(got, ref)


def test_shared_expert_gate_is_sigmoid_of_quant_dot(orc):
    S, t = 5, Q8_0
    spec, h, d, ff = _shared_case(orc, S, t, seed=3)
    gi = orc.normal(77, d, 0.0, 0.05)
    y = orc.shared_expert_add(np.zeros((S, d), np.float32), h, d, ff, (t, t, t), spec.gate[0], spec.up[0],
                              spec.down[0], None)
    base = orc.normal(78, S * d).reshape(S, d)
    got = orc.shared_expert_add(base, h, d, ff, (t, t, t), spec.gate[0], spec.up[0], spec.down[0], gi)
    g = 1.0 / (1.0 + np.exp(-(h.astype(np.float64) @ gi.astype(np.float64))))
    want = base.astype(np.float64) + g[:, None] * y.astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
