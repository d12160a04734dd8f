"""Layer-level parity: kmoe_moe_ffn (Transformer::moe_ffn, transformer.rs:513-570)
against the oracle, and the HBM expert tier's API behaviour."""
import numpy as np
import pytest

from tests.helpers import Q4_K, Q6_K, Q8_0, LayerSpec, random_blocks, rel_l2, row_bytes

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


_layer_id = [100]


def run_layer(ctx, orc, spec: LayerSpec, S: int, regime: int, seed: int, h=None):
    lid = _layer_id[0]
    _layer_id[0] += 1
    spec.upload(ctx, lid)
    try:
        if h is None:
            h = orc.normal(seed, S * spec.d).reshape(S, spec.d)
        ctx.set_regime(regime)
        out = host(ctx.moe_ffn(lid, dev(h)))
        idx, w, perm, off = (host(t) for t in ctx.last_routing(S, spec.k, spec.n_expert))
    finally:
        ctx.set_regime(0)
        ctx.layer_destroy(lid)
    L = spec.oracle_layer()
    ridx, rw = L.route(h, regime)
    rperm, roff = orc.dispatch(ridx, spec.n_expert)
    ref = L.moe_ffn(h, regime)
    return dict(out=out, ref=ref, idx=idx.view(np.uint32), ridx=ridx, w=w, rw=rw, perm=perm.view(np.uint32),
                rperm=rperm, off=off.view(np.uint32), roff=roff)


def check(r, tol=TOL):
    assert np.array_equal(r["idx"], r["ridx"]), "routing indices differ"
    assert np.allclose(r["w"], r["rw"], rtol=1e-6, atol=0), "routing weights differ"
    assert np.array_equal(r["perm"], r["rperm"]), "dispatch permutation differs"
    assert np.array_equal(r["off"], r["roff"]), "dispatch offsets differ"
    e = rel_l2(r["out"], r["ref"])
    assert e < tol, f"rel L2 {e:.3e}"
    return e


@pytest.mark.parametrize("E,K,d,F,S", [(8, 2, 2048, 1024, 16), (8, 2, 2048, 6144, 32), (16, 4, 2048, 768, 24),
                                       (8, 2, 4096, 1024, 8)])
def test_f32_regime_few_rows_is_fp32_accurate(ctx, orc, E, K, d, F, S):
    """The exact regime's experts (every one on the f32 path, at most 32 rows
    each) run the few-rows kernels, whose products use the bf16 matrix cores
    on q and a three-piece split of x: still fp32 accuracy against the
    oracle's f32 dequant-and-multiply, far inside the 1e-3 layer bound;
    gate/up with 1024 rows (two waves per row tile over the superblocks) and
    6144 rows (one wave per row tile), 16 and 17-32 token rows."""
    spec = LayerSpec(E, K, d, F, Q4_K, seed=E + F)
    ctx.profile_enable(True)
    try:
        r = run_layer(ctx, orc, spec, S, 2, seed=S)
        assert ctx.profile_read("moe_gate_up_f32_rows")[1] == 1
        assert ctx.profile_read("moe_down_f32_rows")[1] == 1
    finally:
        ctx.profile_enable(False)
    assert check(r) < 3e-6


@pytest.mark.parametrize("regime", [0, 1, 2])
def test_c1_q8_0_moe_16_tokens(ctx, orc, regime):
    """Config 1: hidden 1024, FFN 512, 8 experts, top-2, Q8_0 from N(0, 0.02),
    16 tokens N(0, 1), seed 0. Under the AVX2 regime experts with >= 4 rows
    take the f32 path and the rest the int8 path, as on the reference host."""
    spec = LayerSpec(8, 2, 1024, 512, Q8_0, seed=0)
    check(run_layer(ctx, orc, spec, 16, regime, seed=0))


@pytest.mark.parametrize("S", [1, 2, 3, 5, 8, 32])
def test_q4k_moe_small_all_regimes(ctx, orc, S):
    spec = LayerSpec(8, 2, 1024, 768, Q4_K, seed=S)
    for regime in (0, 1, 2):
        check(run_layer(ctx, orc, spec, S, regime, seed=1000 + S))


@pytest.mark.parametrize("S", [1, 3, 8, 32])
def test_q4k_m_layer_with_q6k_down(ctx, orc, S):
    """Q4_K_M files keep about half of the ffn_down tensors in Q6_K: Q4_K gate
    and up (tiled in the tier), Q6_K down (GGUF bytes), every regime."""
    spec = LayerSpec(8, 2, 1024, 768, Q4_K, seed=50 + S, down_type=Q6_K)
    for regime in (0, 1, 2):
        check(run_layer(ctx, orc, spec, S, regime, seed=3000 + S))


@pytest.mark.parametrize("S", [1, 5, 16])
def test_q6k_layer_all_parts(ctx, orc, S):
    spec = LayerSpec(8, 2, 1024, 512, Q6_K, seed=60 + S)
    for regime in (0, 1, 2):
        check(run_layer(ctx, orc, spec, S, regime, seed=3100 + S))


def test_mixtral_shape_decode_b1_q6k_down(ctx, orc):
    """Config 3 geometry at decode batch 1 with the Q6_K down projections of a
    Q4_K_M file (split-K down over 210-byte superblocks)."""
    spec = LayerSpec(8, 2, 4096, 14336, Q4_K, seed=5, quantized=False, down_type=Q6_K)
    check(run_layer(ctx, orc, spec, 1, 0, seed=14))


@pytest.mark.parametrize("d,S", [(4096, 2), (4096, 4), (4096, 8), (4096, 16), (8192, 3), (8192, 6)])
def test_few_rows_per_expert_kernels(ctx, orc, d, S):
    """Decode batches: experts with 1..8 rows (1..4 at hidden 8192, two tasks
    per lane) take the register-resident few-rows kernels over tiled Q4_K
    rows; experts with more rows take the matrix-core or LDS-staged kernels in
    the same layer. Both int regimes (AVX2: rows < 4 only)."""
    spec = LayerSpec(8, 2, d, 8192, Q4_K, seed=70 + S, quantized=False)
    for regime in (0, 1):
        check(run_layer(ctx, orc, spec, S, regime, seed=3200 + S))


def test_few_rows_kernels_with_q6k_down(ctx, orc):
    spec = LayerSpec(8, 2, 4096, 8192, Q4_K, seed=81, quantized=False, down_type=Q6_K)
    check(run_layer(ctx, orc, spec, 6, 1, seed=3300))


def test_qwen3_like_zipf_routing(ctx, orc):
    """Config 4 geometry (hidden 2048, FFN 768, 128 experts, top-8, Q4_K) with
    Zipf(1.1) load imbalance; activations offset by +1 carry the bias."""
    spec = LayerSpec(128, 8, 2048, 768, Q4_K, seed=4, quantized=False, zipf=1.1)
    for S, regime in [(1, 0), (16, 0), (64, 1)]:
        h = orc.normal(40 + S, S * 2048, 1.0, 1.0).reshape(S, 2048)
        r = check(run_layer(ctx, orc, spec, S, regime, seed=0, h=h))
        assert r < TOL


_SPECS = {}


def mixtral_spec():
    """Config 3's layer (hidden 4096, FFN 14336, 8 experts, top-2, Q4_K random
    blocks, 793 MB), built once per module."""
    if "mixtral" not in _SPECS:
        _SPECS["mixtral"] = LayerSpec(8, 2, 4096, 14336, Q4_K, seed=3, quantized=False)
    return _SPECS["mixtral"]


def test_mixtral_shape_decode_b1(ctx, orc):
    """Config 3 at decode batch 1: hidden 4096, FFN 14336, 8 experts, top-2,
    Q4_K random blocks (793 MB of experts), router N(0, 0.02)."""
    check(run_layer(ctx, orc, mixtral_spec(), 1, 0, seed=11))


def test_mixtral_shape_prefill_512_int8(ctx, orc):
    """Config 3 at 512 tokens on the int path for every row (the int8
    matrix-core kernels): about 128 rows per expert, so some experts take a
    second 128-row pass."""
    r = run_layer(ctx, orc, mixtral_spec(), 512, 1, seed=12)
    counts = np.diff(r["off"].astype(np.int64))
    assert counts.max() > 128, counts
    check(r)


@pytest.mark.parametrize("S,regime", [(8, 0), (8, 1), (32, 0), (32, 1), (512, 0)])
def test_mixtral_shape_at_bench_token_counts(ctx, orc, S, regime):
    """Config 3 at the token counts the bench reports: decode batches of 8
    and 32 in the AVX2 regime (f32 GEMM for experts with >= 4 rows,
    quant.rs:242-260; the int8 path below) and the int8 regime (few-rows and
    matrix-core kernels), and the 512-token prefill in the AVX2 regime (the
    reference's own prefill arithmetic: every expert on the f32 GEMM)."""
    r = run_layer(ctx, orc, mixtral_spec(), S, regime, seed=4000 + S)
    check(r)


@pytest.mark.parametrize("S,regime", [(512, 0), (512, 1), (2048, 0), (2048, 1)])
def test_qwen3_shape_zipf_at_bench_token_counts(ctx, orc, S, regime):
    """Config 4 (hidden 2048, FFN 768, 128 experts, top-8, Q4_K, Zipf(1.1)
    routing) at the bench's prefill token counts, both regimes."""
    if "qwen3" not in _SPECS:
        _SPECS["qwen3"] = LayerSpec(128, 8, 2048, 768, Q4_K, seed=4, quantized=False, zipf=1.1)
    h = orc.normal(41 + S, S * 2048, 1.0, 1.0).reshape(S, 2048)
    r = run_layer(ctx, orc, _SPECS["qwen3"], S, regime, seed=0, h=h)
    counts = np.diff(r["off"].astype(np.int64))
    assert counts.max() > 4 * max(1, counts.min()), counts  # the Zipf bias skews the expert loads
    check(r)


C5_SHARED_FF = 2816  # 2 shared experts of FFN 1408, stored as one *_shexp FFN


def c5_spec():
    """DeepSeek-V2-Lite-shaped MoE layer (config 5's layer): hidden 2048, 64
    routed experts of FFN 1408, top-6, softmax weights not renormalised
    (norm_topk_prob false, routed scaling 1), Q4_K gate/up and Q8_0 routed
    down (1408 columns need a 32-element block type); the 2 shared experts as
    kestrel holds them, one ffn_*_shexp FFN of width 2816 with no gate
    (scale 1, transformer.rs:572-587), Q4_K gate/up and Q6_K down."""
    if "c5" not in _SPECS:
        spec = LayerSpec(64, 6, 2048, 1408, Q4_K, seed=55, quantized=False, down_type=Q8_0, norm_topk=False,
                         weights_scale=1.0)
        sh = [random_blocks(Q4_K, C5_SHARED_FF, 2048, 901), random_blocks(Q4_K, C5_SHARED_FF, 2048, 902),
              random_blocks(Q6_K, 2048, C5_SHARED_FF, 903)]
        _SPECS["c5"] = (spec, sh)
    return _SPECS["c5"]


@pytest.mark.parametrize("S", [1, 8, 128])
@pytest.mark.parametrize("regime", [0, 1, 2])
def test_c5_deepseek_v2_lite_layer(ctx, orc, S, regime):
    spec, sh = c5_spec()
    lid = _layer_id[0]
    _layer_id[0] += 1
    spec.upload(ctx, lid)
    try:
        ctx.shared_expert(lid, C5_SHARED_FF, (Q4_K, Q4_K, Q6_K), sh[0], sh[1], sh[2], None)
        h = orc.normal(70 + S, S * 2048).reshape(S, 2048)
        ctx.set_regime(regime)
        out = host(ctx.moe_ffn(lid, dev(h)))
        idx, w, perm, off = (host(t) for t in ctx.last_routing(S, spec.k, spec.n_expert))
    finally:
        ctx.set_regime(0)
        ctx.layer_destroy(lid)
    L = spec.oracle_layer()
    ridx, rw = L.route(h, regime)
    rperm, roff = orc.dispatch(ridx, spec.n_expert)
    ref = orc.shared_expert_add(L.moe_ffn(h, regime), h, 2048, C5_SHARED_FF, (Q4_K, Q4_K, Q6_K), sh[0], sh[1], sh[2],
                                None, regime)
    check(dict(out=out, ref=ref, idx=idx.view(np.uint32), ridx=ridx, w=w, rw=rw, perm=perm.view(np.uint32),
               rperm=rperm, off=off.view(np.uint32), roff=roff))
    assert not np.allclose(rw.sum(1), 1.0)  # no renormalisation: the six weights sum below 1


@pytest.mark.parametrize("S,E,k", [(300, 4, 2), (129, 2, 2), (9, 16, 4)])
def test_q4k_moe_int8_token_passes(ctx, orc, S, E, k):
    """Grouped int8 path with experts of 0, few and more than 128 rows (token
    passes of 128), and every token on both experts when E == k."""
    spec = LayerSpec(E, k, 512, 768, Q4_K, seed=S)
    check(run_layer(ctx, orc, spec, S, 1, seed=2000 + S))


@pytest.mark.parametrize("d,S", [(4096, 1), (1024, 1), (1024, 2), (1024, 6)])
def test_nan_router_row_routes_in_index_order(ctx, orc, d, S):
    """A NaN router weight: every p of every token is NaN, and the reference
    selects experts 0..k-1 (transformer.rs:479-484). One token selects inside
    the gate/up kernel (tiled Q4_K rows at d = 4096, the register kernel at
    1024); more tokens go through the router kernels. The output is NaN."""
    spec = LayerSpec(8, 2, d, 512, Q4_K, seed=4, quantized=False)
    spec.router[5, 17] = np.nan
    r = run_layer(ctx, orc, spec, S, 0, seed=77)
    assert r["ridx"].tolist() == [[0, 1]] * S
    assert np.array_equal(r["idx"], r["ridx"])
    assert np.array_equal(r["perm"], r["rperm"]) and np.array_equal(r["off"], r["roff"])
    assert np.isnan(r["w"]).all() and np.isnan(r["out"]).all() and np.isnan(r["ref"]).all()


def test_norm_topk_off_and_weights_scale(ctx, orc):
    spec = LayerSpec(16, 4, 1024, 512, Q8_0, seed=9, norm_topk=False, weights_scale=2.5)
    check(run_layer(ctx, orc, spec, 6, 0, seed=3))


# ----------------------------------------------------------------- expert tier
def test_expert_tier_serves_correct_slices(ctx):
    """memory/src/expert.rs:731-751: every expert slice holds l*1000 + e*10 + k;
    the tier must hand back exactly those bytes for (layer, expert, part)."""
    import ctypes

    d, ff, E = 256, 256, 8
    for l in range(2):
        ctx.layer_create(l, E, 2, d, ff, Q8_0, Q8_0, Q8_0)
        assert not ctx.expert_is_ready(l, 0)
        for e in range(E):
            for k in range(3):
                n = row_bytes(Q8_0, d if k < 2 else ff) * (ff if k < 2 else d)
                v = np.full(n // 4, l * 1000 + e * 10 + k, np.float32)
                ctx.expert_upload(l, e, k, v.view(np.uint8))
        for e in range(E):
            assert ctx.expert_is_ready(l, e)
            for k in range(3):
                p, n = ctx.expert_part(l, e, k)
                buf = np.empty(n // 4, np.float32)
                ctx.check(ctx.lib.kmoe_copy_d2h(ctx.h, buf.ctypes.data, ctypes.c_void_p(p), n))
                assert np.all(buf == l * 1000 + e * 10 + k)
            for k in range(3):
                assert np.all(ctx.expert_read(l, e, k).view(np.float32) == l * 1000 + e * 10 + k)
        assert ctx.bytes_per_expert(l) == 3 * 256 * 8 * 34
    ctx.layer_destroy(0)
    ctx.layer_destroy(1)


@pytest.mark.parametrize("S,regime", [(1, 0), (3, 0), (6, 0), (6, 1)])
def test_moe_ffn_host_is_moe_ffn(ctx, orc, S, regime):
    """kmoe_moe_ffn_host, moe_ffn's own signature (transformer.rs:513: h:
    &[f32] in, Vec<f32> out): the same bits as kmoe_moe_ffn on device buffers."""
    spec = LayerSpec(8, 2, 4096, 1024, Q4_K, seed=31, quantized=False, down_type=Q6_K)
    lid = _layer_id[0]
    _layer_id[0] += 1
    spec.upload(ctx, lid)
    try:
        ctx.set_regime(regime)
        h = orc.normal(40 + S, S * 4096).reshape(S, 4096)
        a = ctx.moe_ffn_host(lid, h)
        b = host(ctx.moe_ffn(lid, dev(h)))
    finally:
        ctx.set_regime(0)
        ctx.layer_destroy(lid)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert rel_l2(a, spec.oracle_layer().moe_ffn(h, regime)) < TOL


def test_tiled_parts_report_their_layout_and_raw_kernels_refuse_them(ctx):
    """kmoe_expert_part hands out tier bytes in the tier's layout: Q4_K and
    Q6_K parts are tiled rows, Q8_0 parts GGUF bytes. The raw-pointer entry
    points read GGUF rows, so they refuse a pointer to a tiled part instead
    of returning wrong numbers; a GGUF (Q8_0) part still works."""
    import torch

    from kestrel_amd.kmoe import KmoeError

    spec = LayerSpec(2, 1, 1024, 512, Q4_K, seed=5, quantized=False, down_type=Q8_0)
    lid = _layer_id[0]
    _layer_id[0] += 1
    spec.upload(ctx, lid)
    try:
        assert [ctx.expert_part_layout(lid, 1, k) for k in range(3)] == [1, 1, 0]
        x = torch.ones((1, 1024), dtype=torch.float32, device="cuda")
        p, n = ctx.expert_part(lid, 1, 0)
        rc = ctx.lib.kmoe_matmul(ctx.h, Q4_K, p, n, 512, 1024, x.data_ptr(), 1, x.data_ptr())
        assert rc == -1 and b"tiled" in ctx.lib.kmoe_last_error(ctx.h)
        with pytest.raises(KmoeError):
            ctx.matmul_host(Q4_K, _DevBuf(p, n), 512, 1024, np.ones((1, 1024), np.float32))
        p2, n2 = ctx.expert_part(lid, 1, 2)  # Q8_0 down [1024, 512]: GGUF bytes, usable as is
        y = ctx.matmul_host(Q8_0, _DevBuf(p2, n2), 1024, 512, np.ones((1, 512), np.float32))
        ref = ctx.matmul_host(Q8_0, spec.down[1], 1024, 512, np.ones((1, 512), np.float32))
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    finally:
        ctx.layer_destroy(lid)


class _DevBuf:
    """A raw device pointer with the two methods Context.matmul_host reads."""

    def __init__(self, p, n):
        self.p, self.n = p, n

    def data_ptr(self):
        return self.p

    def numel(self):
        return self.n

    def element_size(self):
        return 1


def _tiled_reference(g: np.ndarray, rows: int, nb: int) -> np.ndarray:
    """Tiled Q4_K rows written out chunk by chunk from the layout's definition:
    heads first, then per group of 8 superblocks the chunks (j, superblock, k)."""
    out = np.empty_like(g)
    for r in range(rows):
        row = g[r * 144 * nb:(r + 1) * 144 * nb].reshape(nb, 144)
        parts = [row[:, :16].reshape(-1)]
        for g0 in range(0, nb, 8):
            sbs = row[g0:min(nb, g0 + 8), 16:].reshape(-1, 4, 2, 16)  # (superblock, k, j, 16 bytes)
            parts.append(sbs.transpose(2, 0, 1, 3).reshape(-1))
        out[r * 144 * nb:(r + 1) * 144 * nb] = np.concatenate(parts)
    return out


@pytest.mark.parametrize("d,ff", [(4096, 512), (1024, 14336 // 7), (768, 2304)])
def test_q4k_tier_layout_round_trip(ctx, d, ff):
    """Q4_K parts are stored as tiled rows: host and device uploads produce the
    same bytes, the layout matches its definition (heads, then 8-superblock
    groups, partial last group included), and kmoe_expert_read restores GGUF."""
    import ctypes

    import torch

    rng = np.random.default_rng(d + ff)
    ctx.layer_create(95, 4, 2, d, ff, Q4_K, Q4_K, Q4_K)
    try:
        for p in range(3):
            rows, nb = (ff, d // 256) if p < 2 else (d, ff // 256)
            g = rng.integers(0, 256, rows * nb * 144, dtype=np.uint8)
            ctx.expert_upload(95, 0, p, g)
            ctx.expert_upload(95, 1, p, torch.from_numpy(g).cuda())
            for e in (0, 1):
                ptr, n = ctx.expert_part(95, e, p)
                raw = np.empty(n, np.uint8)
                ctx.check(ctx.lib.kmoe_copy_d2h(ctx.h, raw.ctypes.data, ctypes.c_void_p(ptr), n))
                assert np.array_equal(raw, _tiled_reference(g, rows, nb)), (p, e)
                assert np.array_equal(ctx.expert_read(95, e, p), g), (p, e)
    finally:
        ctx.layer_destroy(95)


def _tiled_q6k_reference(g: np.ndarray, rows: int, nb: int) -> np.ndarray:
    """Tiled Q6_K rows from the layout's definition: task k = 2h + p of a
    superblock takes nibble p of ql[64h + b] (low) and ql[64h + 32 + b] (high)
    for b < 32, and bits 4p..4p+3 of qh[32h + b] (low) and qh[32h + 16 + b]
    (high) for b < 16; per group of 8 superblocks the 16-byte pieces
    (j, superblock, k); then the scale bytes, then d."""
    out = np.empty_like(g)
    for r in range(rows):
        blk = g[r * 210 * nb:(r + 1) * 210 * nb].reshape(nb, 210)
        ql = blk[:, :128].reshape(nb, 2, 64)
        qh = blk[:, 128:192].reshape(nb, 2, 32)
        P = np.empty((nb, 4, 3, 16), np.uint8)
        for k in range(4):
            h, p = k >> 1, k & 1
            nib = lambda v: (v >> 4) if p else (v & 0xF)
            n = nib(ql[:, h, :32]) | (nib(ql[:, h, 32:]) << 4)
            P[:, k, 0], P[:, k, 1] = n[:, :16], n[:, 16:]
            P[:, k, 2] = ((qh[:, h, :16] >> (4 * p)) & 0xF) | (((qh[:, h, 16:] >> (4 * p)) & 0xF) << 4)
        parts = [P[g0:min(nb, g0 + 8)].transpose(2, 0, 1, 3).reshape(-1) for g0 in range(0, nb, 8)]
        parts += [blk[:, 192:208].reshape(-1), blk[:, 208:210].reshape(-1)]
        out[r * 210 * nb:(r + 1) * 210 * nb] = np.concatenate(parts)
    return out


@pytest.mark.parametrize("d,ff", [(4096, 512), (1024, 14336 // 7), (768, 2304)])
def test_q6k_tier_layout_round_trip(ctx, d, ff):
    """Q6_K parts are stored as tiled rows (per-task nibble and high-bit pieces):
    host and device uploads agree with the layout's definition, partial groups
    and odd superblock counts included, and kmoe_expert_read restores GGUF."""
    import ctypes

    import torch

    rng = np.random.default_rng(d * 3 + ff)
    ctx.layer_create(96, 4, 2, d, ff, Q6_K, Q6_K, Q6_K)
    try:
        for p in range(3):
            rows, nb = (ff, d // 256) if p < 2 else (d, ff // 256)
            g = rng.integers(0, 256, rows * nb * 210, dtype=np.uint8)
            ctx.expert_upload(96, 0, p, g)
            ctx.expert_upload(96, 1, p, torch.from_numpy(g).cuda())
            for e in (0, 1):
                ptr, n = ctx.expert_part(96, e, p)
                raw = np.empty(n, np.uint8)
                ctx.check(ctx.lib.kmoe_copy_d2h(ctx.h, raw.ctypes.data, ctypes.c_void_p(ptr), n))
                assert np.array_equal(raw, _tiled_q6k_reference(g, rows, nb)), (p, e)
                assert np.array_equal(ctx.expert_read(96, e, p), g), (p, e)
    finally:
        ctx.layer_destroy(96)


def _tier_bytes(ctx, layer, E):
    import ctypes

    out = []
    for e in range(E):
        for k in range(3):
            p, n = ctx.expert_part(layer, e, k)
            raw = np.empty(n, np.uint8)
            ctx.check(ctx.lib.kmoe_copy_d2h(ctx.h, raw.ctypes.data, ctypes.c_void_p(p), n))
            out.append(raw)
    return out


def _ffn(ctx, layer, h):
    return host(ctx.moe_ffn(layer, dev(h)))


@pytest.mark.parametrize("wtype,down,d,ff", [(Q4_K, Q6_K, 512, 768), (Q8_0, Q8_0, 256, 512),
                                             (Q6_K, Q4_K, 256, 1280)])
def test_prepared_layout_preloads_identical_experts_in_one_copy(ctx, orc, wtype, down, d, ff):
    """expert.rs:755-777: a prepared container serves the same experts as the
    plain GGUF in one read per expert instead of three. Here the whole layer
    is preloaded (preload_all) from both images: one host-to-device copy per
    expert from the KGUF, three from the GGUF, and the tier, kmoe_expert_read
    and the layer's output are identical to part-by-part uploads."""
    from tests.helpers import expert_images

    E = 8
    spec = LayerSpec(E, 2, d, ff, wtype, seed=31, down_type=down)
    (plain, (poff, pstride)), (kg, (koff, kstride)) = expert_images(spec, seed=31)
    ids = (140, 141, 142)
    spec.upload(ctx, ids[0])
    try:
        for lid in ids[1:]:
            ctx.layer_create(lid, E, 2, d, ff, wtype, wtype, down)
            ctx.router_upload(lid, spec.router)
            assert not ctx.expert_is_ready(lid, 0)
        assert ctx.layer_preload(ids[1], plain, poff, pstride) == 3 * E
        assert ctx.layer_preload(ids[2], kg, koff, kstride) == E
        want = _tier_bytes(ctx, ids[0], E)
        for lid in ids[1:]:
            assert all(ctx.expert_is_ready(lid, e) for e in range(E))
            got = _tier_bytes(ctx, lid, E)
            assert all(np.array_equal(a, b) for a, b in zip(got, want)), lid
            for e in range(E):
                for k, src in enumerate((spec.gate, spec.up, spec.down)):
                    assert np.array_equal(ctx.expert_read(lid, e, k), src[e]), (lid, e, k)
        h = orc.normal(8, 5 * d).reshape(5, d)
        outs = [_ffn(ctx, lid, h) for lid in ids]
        assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
        assert rel_l2(outs[2], spec.oracle_layer().moe_ffn(h, 0)) < TOL
    finally:
        for lid in ids:
            ctx.layer_destroy(lid)


@pytest.mark.parametrize("wtype,down", [(Q4_K, Q6_K), (Q8_0, Q4_K)])
def test_expert_buffer_upload_one_copy(ctx, orc, wtype, down):
    """ExpertBuf (expert.rs:62-76): the extents of one expert in one host
    buffer, parts at arbitrary positions (odd ones included, as a head offset
    inside an aligned read gives) and in file order rather than part order;
    the tier holds what part-by-part uploads give."""
    E, d, ff = 4, 256, 512
    spec = LayerSpec(E, 2, d, ff, wtype, seed=41, down_type=down)
    rng = np.random.default_rng(41)
    spec.upload(ctx, 143)
    ctx.layer_create(144, E, 2, d, ff, wtype, wtype, down)
    ctx.router_upload(144, spec.router)
    try:
        for e in range(E):
            g, u, dn = spec.gate[e], spec.up[e], spec.down[e]
            pos_down = 4096 + 2 * e + 1
            pos_gate = pos_down + len(dn) + 4000 + 3
            pos_up = pos_gate + len(g) + 17
            buf = rng.integers(0, 256, pos_up + len(u) + 4096, dtype=np.uint8)
            buf[pos_gate:pos_gate + len(g)] = g
            buf[pos_up:pos_up + len(u)] = u
            buf[pos_down:pos_down + len(dn)] = dn
            ctx.expert_upload_buf(144, e, buf, (pos_gate, pos_up, pos_down))
            assert ctx.expert_is_ready(144, e)
        want, got = _tier_bytes(ctx, 143, E), _tier_bytes(ctx, 144, E)
        assert all(np.array_equal(a, b) for a, b in zip(got, want))
        h = orc.normal(9, 3 * d).reshape(3, d)
        assert np.array_equal(_ffn(ctx, 143, h), _ffn(ctx, 144, h))
    finally:
        ctx.layer_destroy(143)
        ctx.layer_destroy(144)


def test_uploads_without_room_for_staging_go_part_by_part(orc):
    """With the VRAM budget (ledger.rs:75-102) too tight for the upload
    staging, the uploads still succeed part by part (tiled on the host) and
    stay within the budget: the staging is an optimisation, never an error."""
    from kestrel_amd.kmoe import Context
    from tests.helpers import expert_images

    E, d, ff = 4, 256, 512
    spec = LayerSpec(E, 2, d, ff, Q4_K, seed=51, down_type=Q6_K)
    _, (kg, (koff, kstride)) = expert_images(spec, seed=51)
    c = Context(0)
    try:
        base, _ = c.vram_usage()
        c.layer_create(1, E, 2, d, ff, Q4_K, Q4_K, Q6_K)
        after, _ = c.vram_usage()
        c.vram_set_limit(after + 4096)
        c.router_upload(1, spec.router)
        assert c.layer_preload(1, kg, koff, kstride) == 3 * E
        for e in range(E):
            for k, src in enumerate((spec.gate, spec.up, spec.down)):
                assert np.array_equal(c.expert_read(1, e, k), src[e]), (e, k)
        buf = np.concatenate([spec.gate[0], spec.up[0], spec.down[0]])
        c.expert_upload_buf(1, 0, buf, (0, len(spec.gate[0]), len(spec.gate[0]) + len(spec.up[0])))
        c.expert_upload(1, 1, 2, spec.down[1])
        assert c.vram_usage()[0] <= after + 4096
        c.vram_set_limit(0)  # room for the moe_ffn workspace
        h = orc.normal(10, 2 * d).reshape(2, d)
        out = host(c.moe_ffn(1, dev(h)))
        assert rel_l2(out, spec.oracle_layer().moe_ffn(h, 0)) < TOL
        assert base < after
    finally:
        c.sync()
        c.close()


def test_extent_upload_errors(ctx):
    import ctypes

    from kestrel_amd.kmoe import KmoeError

    ctx.layer_create(145, 4, 2, 256, 256, Q4_K, Q4_K, Q4_K)
    try:
        n = row_bytes(Q4_K, 256) * 256
        buf = np.zeros(3 * n, np.uint8)
        with pytest.raises(KmoeError) as e:  # part overruns the buffer
            ctx.expert_upload_buf(145, 0, buf, (0, n, 2 * n + 1))
        assert e.value.status == -1
        with pytest.raises(KmoeError) as e:  # expert out of range
            ctx.expert_upload_buf(145, 4, buf, (0, n, 2 * n))
        assert e.value.status == -1
        assert not ctx.expert_is_ready(145, 0)
        with pytest.raises(ValueError):  # the image ends before expert 3's parts
            ctx.layer_preload(145, np.zeros(4 * n, np.uint8), (0, n, 2 * n), (3 * n,) * 3)
        strides = (ctypes.c_uint64 * 3)(n, n, n)
        bases = (ctypes.c_void_p * 3)(buf.ctypes.data, None, buf.ctypes.data)
        assert ctx.lib.kmoe_layer_preload(ctx.h, 145, bases, strides, None) == -1
        assert ctx.lib.kmoe_layer_preload(ctx.h, 999, bases, strides, None) == -5
    finally:
        ctx.layer_destroy(145)


def test_errors_map_to_status_codes(ctx):
    from kestrel_amd.kmoe import KmoeError

    import torch

    w = torch.zeros(10, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(KmoeError) as e:  # weight buffer smaller than rows x row_bytes (quant.rs:233-234)
        ctx.matmul(Q4_K, w, 4, 256, x)
    assert e.value.status == -1
    with pytest.raises(KmoeError) as e:  # a type quant::matmul does not take either (Q3_K, quant.rs:48-51)
        ctx.matmul(11, w, 4, 256, x)
    assert e.value.status == -2
    with pytest.raises(KmoeError) as e:  # layer never created
        ctx.moe_ffn(77, x)
    assert e.value.status == -5
    ctx.layer_create(78, 8, 2, 256, 256, Q4_K, Q4_K, Q4_K)
    with pytest.raises(KmoeError) as e:  # experts not resident
        ctx.moe_ffn(78, x)
    assert e.value.status == -5
    ctx.layer_destroy(78)
    reserved, limit = ctx.vram_usage()
    ctx.vram_set_limit(reserved + 1024)
    try:
        with pytest.raises(KmoeError) as e:  # Tier::Vram budget (ledger.rs:75-102)
            ctx.layer_create(79, 8, 2, 4096, 14336, Q4_K, Q4_K, Q4_K)
        assert e.value.status == -3
    finally:
        ctx.vram_set_limit(0)


def test_device_generated_weights_are_stream_ordered(ctx, orc):
    """Weights written by torch kernels on its current stream and uploaded at
    once (no host sync) must be what the kernels read: the library runs on
    torch's stream, including the null stream."""
    import ctypes

    import torch

    d, ff, E, k = 1024, 768, 8, 2
    ctx.layer_create(90, E, k, d, ff, Q4_K, Q4_K, Q4_K)
    hdr = torch.tensor(np.concatenate([np.array([1.4e-4], np.float16).view(np.uint8),
                                       np.array([1.05e-3], np.float16).view(np.uint8)]), device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    for e in range(E):
        for p in range(3):
            n = ff * row_bytes(Q4_K, d) if p < 2 else d * row_bytes(Q4_K, ff)
            t = torch.randint(0, 256, (n // 144, 144), dtype=torch.uint8, device="cuda", generator=g)
            t[:, 0:4] = hdr
            ctx.expert_upload(90, e, p, t)
            del t
    router = orc.normal(3, E * d, 0.0, 0.02).reshape(E, d)
    ctx.router_upload(90, router)
    gh = torch.Generator(device="cuda")
    gh.manual_seed(7)  # a fixed input: an unseeded one can land an int8 rounding of h on a midpoint
    h = torch.randn((4, d), device="cuda", generator=gh) * 2.0  # async producer right before the call
    out = host(ctx.moe_ffn(90, h))
    parts = [[None] * 3 for _ in range(E)]
    for e in range(E):
        for p in range(3):
            buf = ctx.expert_read(90, e, p)
            assert np.all(buf.reshape(-1, 144)[:, :4] == hdr.cpu().numpy()), (e, p)
            parts[e][p] = buf
    ctx.layer_destroy(90)
    L = orc.Layer(E, k, d, ff, Q4_K, Q4_K, Q4_K, router, [p[0] for p in parts], [p[1] for p in parts],
                  [p[2] for p in parts], True, 0.0)
    ref = L.moe_ffn(h.cpu().numpy())
    assert np.isfinite(out).all()
    assert rel_l2(out, ref) < TOL


# --------------------------------------------------------------- shared expert
@pytest.mark.parametrize("wtype,ffs", [(Q8_0, 1024), (Q4_K, 1536)])
@pytest.mark.parametrize("with_gate", [False, True])
def test_shared_expert_layer(ctx, orc, wtype, ffs, with_gate):
    """qwen2moe layer (transformer.rs:572-587): routed experts plus a shared
    expert scaled by sigmoid(quant::dot(ffn_gate_inp_shexp, h)) or 1."""
    d, ff = 1024, 512
    spec = LayerSpec(8, 2, d, ff, wtype, seed=31 + wtype)
    sh = [orc.quantize(wtype, orc.normal(900 + p, (ffs * d), 0.0, 0.02).reshape(*((ffs, d) if p < 2 else (d, ffs))))
          for p in range(3)]
    gi = orc.normal(950, d, 0.0, 0.05) if with_gate else None
    L = spec.oracle_layer()
    for S, regime in [(1, 0), (3, 0), (6, 0), (5, 1), (4, 2)]:
        lid = _layer_id[0]
        _layer_id[0] += 1
        spec.upload(ctx, lid)
        try:
            ctx.shared_expert(lid, ffs, (wtype, wtype, wtype), sh[0], sh[1], sh[2], gi)
            h = orc.normal(960 + S, S * d).reshape(S, d)
            ctx.set_regime(regime)
            out = host(ctx.moe_ffn(lid, dev(h)))
        finally:
            ctx.set_regime(0)
            ctx.layer_destroy(lid)
        ref = orc.shared_expert_add(L.moe_ffn(h, regime), h, d, ffs, (wtype, wtype, wtype), sh[0], sh[1], sh[2], gi,
                                    regime)
        e = rel_l2(out, ref)
        assert e < TOL, (S, regime, e)


@pytest.mark.parametrize("types,ffs,with_gate,rff,rdown,fused", [
    ((Q4_K, Q4_K, Q6_K), C5_SHARED_FF, False, 1024, None, False),  # DeepSeek-V2-Lite's shared experts
    ((Q4_K, Q4_K, Q6_K), C5_SHARED_FF, False, 1408, Q8_0, True),   # ... with its routed Q8_0 down: one down kernel
    ((Q4_K, Q4_K, Q4_K), 1536, True, 1024, None, False),
    ((Q4_K, Q4_K, Q4_K), 1536, True, 1536, None, True),           # 32 lanes per row on both: one down kernel
    ((Q8_0, Q8_0, Q8_0), 1024, True, 1024, None, False),
])
@pytest.mark.parametrize("regime", [0, 1])
def test_shared_expert_one_token_bits_of_product_sequence(ctx, orc, types, ffs, with_gate, rff, rdown, fused, regime):
    """One token on the int8 path: the shared expert (one product over the
    back-to-back gate and up rows, SwiGLU fused with the quantization of its
    output, down adding its gated result into out) gives the bits of the
    sequence transformer.rs:572-587 spells out, made of separate calls:
    quant::matmul of gate and of up (kmoe_matmul, the same int8 products),
    SwiGLU and sigmoid with a correctly rounded exp, quant::matmul of down, and
    out + scale * y on top of the routed experts' output. Where the routed
    and shared down rows share a launch shape, both run in one kernel (the
    library's timing names it), with the same bits."""
    d = 2048
    t0, _, t2 = types
    spec = LayerSpec(16, 4, d, rff, t0, seed=40 + ffs, quantized=False, down_type=rdown or t0)
    sh = [random_blocks(t0, ffs, d, 910), random_blocks(t0, ffs, d, 911), random_blocks(t2, d, ffs, 912)]
    gi = orc.normal(951, d, 0.0, 0.05) if with_gate else None
    h = orc.normal(952, d).reshape(1, d)
    outs = []
    ctx.set_regime(regime)
    try:
        for shared in (True, False):
            lid = _layer_id[0]
            _layer_id[0] += 1
            spec.upload(ctx, lid)
            try:
                if shared:
                    ctx.shared_expert(lid, ffs, types, sh[0], sh[1], sh[2], gi)
                    ctx.profile_enable(True)
                outs.append(host(ctx.moe_ffn(lid, dev(h))))
                if shared:
                    assert ctx.profile_read("moe_down_shared")[1] == (1 if fused else 0)
            finally:
                ctx.profile_enable(False)
                ctx.layer_destroy(lid)
        g = host(ctx.matmul(t0, dev(sh[0]), ffs, d, dev(h)))
        u = host(ctx.matmul(t0, dev(sh[1]), ffs, d, dev(h)))
        e = np.exp(-g.astype(np.float64)).astype(np.float32)  # correctly rounded up to double rounding
        a = (g / (np.float32(1.0) + e)) * u
        y = host(ctx.matmul(t2, dev(sh[2]), d, ffs, dev(a)))
        scale = np.float32(1.0)
        if with_gate:
            gl = host(ctx.matmul(0, dev(gi), 1, d, dev(h)))[0, 0]
            scale = np.float32(1.0) / (np.float32(1.0) + np.float32(np.exp(-np.float64(gl))))
    finally:
        ctx.set_regime(0)
    exp = outs[1] + scale * y
    assert np.array_equal(outs[0].view(np.uint32), exp.view(np.uint32)), \
        int((outs[0].view(np.uint32) != exp.view(np.uint32)).sum())
    ref = orc.shared_expert_add(spec.oracle_layer().moe_ffn(h, regime), h, d, ffs, types, sh[0], sh[1], sh[2], gi,
                                regime)
    assert rel_l2(outs[0], ref) < TOL


def test_shared_expert_errors(ctx):
    from kestrel_amd.kmoe import KmoeError

    ctx.layer_create(97, 8, 2, 256, 256, Q8_0, Q8_0, Q8_0)
    try:
        with pytest.raises(KmoeError) as e:  # gate vector before the shared expert exists
            ctx.check(ctx.lib.kmoe_shared_gate_upload(ctx.h, 97, None, 0))
        assert e.value.status == -5
        ctx.check(ctx.lib.kmoe_shared_expert_create(ctx.h, 97, 512, Q8_0, Q8_0, Q8_0))
        with pytest.raises(KmoeError) as e:  # wrong part size
            b = np.zeros(10, np.uint8)
            ctx.check(ctx.lib.kmoe_shared_expert_upload(ctx.h, 97, 0, b.ctypes.data, b.nbytes))
        assert e.value.status == -1
    finally:
        ctx.layer_destroy(97)


@pytest.mark.parametrize("wtype,d,ff,S,regime,with_y", [
    (Q4_K, 1024, 1536, 1, 0, True),   # one token: the router kernel takes the norm (Q8_K rows)
    (Q4_K, 1024, 1536, 1, 1, False),  # int8 regime, no residual add
    (Q8_0, 2048, 1024, 1, 0, True),   # Q8 rows for Q8_0 experts
    (Q4_K, 1024, 1536, 1, 2, True),   # exact regime: no int8 rows
    (Q4_K, 1024, 1536, 3, 0, True),   # three tokens: the norm kernel, then the layer
])
def test_norm_moe_ffn_matches_rmsnorm_then_moe(ctx, orc, wtype, d, ff, S, regime, with_y):
    """kmoe_norm_moe_ffn against kmoe_rmsnorm followed by kmoe_moe_ffn on the
    same inputs: x after the residual add, the normed rows f and the layer's
    output are the same bits, called twice in a row."""
    import torch

    spec = LayerSpec(32, 4, d, ff, wtype, seed=d + ff + S, quantized=False)
    lid = _layer_id[0]
    _layer_id[0] += 1
    spec.upload(ctx, lid)
    ctx.set_regime(regime)
    try:
        nw = dev(orc.normal(7 + S, d, 1.0, 0.1))
        for call in range(2):
            x0 = orc.normal(50 + call, S * d, 0.0, 1.0).reshape(S, d)
            y = dev(orc.normal(60 + call, S * d, 0.0, 0.5).reshape(S, d)) if with_y else None
            xa, xb = dev(x0), dev(x0)
            fa = ctx.rmsnorm(xa, nw, 1e-5, y=y)
            a = host(ctx.moe_ffn(lid, fa))
            fb = torch.empty_like(xb)
            b = host(ctx.norm_moe_ffn(lid, xb, nw, 1e-5, y=y, f=fb))
            for u, v in ((host(xa), host(xb)), (host(fa), host(fb)), (a, b)):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), (call, np.abs(u - v).max())
    finally:
        ctx.set_regime(0)
        ctx.layer_destroy(lid)


@pytest.mark.parametrize("shape", ["qwen3_small", "c5_small"])
def test_decode_batches_graph_replays_equal_eager(ctx, orc, shape):
    """Decode batches captured in one HIP graph: the router launch with its
    quantizing work-groups, top-k, dispatch, the few-rows int kernels, the
    f32 kernels (ranked grids, one, two and four token tiles; the shared
    expert's plain-row gate/up) and the combine, at 6, 16, 24 and 40 tokens in
    the AVX2 and int8 regimes. Every replay, with eager calls and
    synchronizations between replays, equals the eager result bit for bit."""
    import torch

    sh = None
    if shape == "qwen3_small":  # narrow rows (the few-rows int kernels), Zipf skew
        spec = LayerSpec(32, 8, 2048, 768, Q4_K, seed=11, quantized=False, zipf=1.1)
    else:  # 64 experts top-6, Q8_0 down, an ungated shared FFN (Q4_K gate/up, Q6_K down)
        spec, sh = c5_spec()
    lid = _layer_id[0]
    _layer_id[0] += 1
    spec.upload(ctx, lid)
    try:
        if sh is not None:
            ctx.shared_expert(lid, C5_SHARED_FF, (Q4_K, Q4_K, Q6_K), sh[0], sh[1], sh[2], None)
        for regime in (0, 1):
            ctx.set_regime(regime)
            xs = [torch.from_numpy(orc.normal(900 + S + 7 * regime, S * spec.d, 1.0, 1.0).reshape(S, spec.d)).cuda()
                  for S in (6, 16, 24, 40)]
            outs = [torch.empty_like(x) for x in xs]
            eager = []
            for x, o in zip(xs, outs):
                ctx.moe_ffn(lid, x, o)
                eager.append(o.clone())
            torch.cuda.synchronize()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                ctx.set_stream(s)
                with torch.cuda.graph(g, stream=s):
                    for x, o in zip(xs, outs):
                        ctx.moe_ffn(lid, x, o)
            torch.cuda.current_stream().wait_stream(s)
            ctx.set_stream(torch.cuda.current_stream())
            for rep in range(3):
                for o in outs:
                    o.zero_()
                g.replay()
                torch.cuda.synchronize()
                for i, (o, e) in enumerate(zip(outs, eager)):
                    assert torch.equal(o, e), (shape, regime, rep, i)
                # eager work between replays
                ctx.moe_ffn(lid, xs[1], torch.empty_like(xs[1]))
                torch.cuda.synchronize()
            del g
    finally:
        ctx.set_regime(0)
        ctx.set_stream(torch.cuda.current_stream())
        ctx.layer_destroy(lid)
