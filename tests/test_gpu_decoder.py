"""The rest of the decoder layer on the GPU (include/kmoe.h decoder ops and
kestrel_amd.decoder) against the oracle's restatement of
Transformer::forward (transformer.rs:278-302, 330-467, 591-631)."""
import numpy as np
import pytest

from tests.helpers import (DSV2LITE, F32, Q4_K, Q6_K, Q8_0, LayerSpec, decoder_model, random_blocks, rel_l2,
                           row_bytes, stack_model)

pytestmark = pytest.mark.gpu

F16 = 1


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


@pytest.mark.parametrize("t,cols", [(F32, 96), (F16, 64), (Q8_0, 320), (Q4_K, 512), (Q6_K, 768)])
def test_get_rows_bit_exact(ctx, orc, t, cols):
    rng = np.random.default_rng(t + cols)
    n_rows = 50
    if t == F32:
        table = rng.standard_normal(n_rows * cols).astype(np.float32).view(np.uint8)
    elif t == F16:
        table = rng.standard_normal(n_rows * cols).astype(np.float16).view(np.uint8)
    else:
        table = random_blocks(t, n_rows, cols, seed=t)
    rb = table.size // n_rows
    ids = [0, 49, 7, 7, 23]
    got = host(ctx.get_rows(t, dev(table), n_rows, cols, ids))
    ref = np.stack([orc.dequant(t, table[i * rb:(i + 1) * rb], cols) for i in ids])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    import torch

    got_dev = host(ctx.get_rows(t, dev(table), n_rows, cols, torch.tensor(ids, dtype=torch.int32).cuda()))
    assert np.array_equal(got_dev.view(np.uint32), ref.view(np.uint32))


def test_get_rows_rejects_out_of_range_ids(ctx):
    from kestrel_amd.kmoe import KmoeError

    table = dev(np.zeros(10 * 34, np.uint8))
    with pytest.raises(KmoeError) as e:  # EngineError "token id out of range" (transformer.rs:384-386)
        ctx.get_rows(Q8_0, table, 10, 32, [3, 10])
    assert e.value.status == -1


@pytest.mark.parametrize("rows,dim", [(1, 4096), (7, 2048), (64, 128)])
def test_rmsnorm_with_residual(ctx, orc, rows, dim):
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal((rows, dim)) * 2).astype(np.float32)
    y = rng.standard_normal((rows, dim)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    got = host(ctx.rmsnorm(dev(x), dev(w), 1e-5))
    assert rel_l2(got, orc.rmsnorm(x, w, 1e-5)) < 1e-6
    xd = dev(x)
    got = host(ctx.rmsnorm(xd, dev(w), 1e-5, y=dev(y)))
    assert np.array_equal(host(xd), x + y)  # the residual add is stored
    assert rel_l2(got, orc.rmsnorm(x + y, w, 1e-5)) < 1e-6
    ctx.rmsnorm(xd, dev(w), 1e-5, out=xd)  # in place
    assert rel_l2(host(xd), orc.rmsnorm(x + y, w, 1e-5)) < 1e-6


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("nh,hd,rd,S,pos0", [(8, 128, 128, 1, 0), (4, 64, 32, 9, 1000), (2, 128, 64, 3, 70000)])
def test_rope(ctx, orc, neox, nh, hd, rd, S, pos0):
    import torch

    rng = np.random.default_rng(nh * S)
    x = rng.standard_normal((S, nh * hd)).astype(np.float32)
    f = orc.rope_inv_freq(10000.0, rd)
    ref = orc.rope(x, nh, hd, rd, pos0, f, neox)
    got = host(ctx.rope(dev(x), nh, hd, rd, pos0, dev(f), neox))
    assert np.abs(got - ref).max() <= 2e-6 * max(1.0, np.abs(ref).max())
    pos = torch.tensor([pos0 - 1], dtype=torch.int32).cuda()
    got2 = host(ctx.rope(dev(x), nh, hd, rd, 1, dev(f), neox, pos_dev=pos))  # device position + pos0
    assert np.array_equal(got2, got)


def test_kv_store_bit_exact_at_host_and_device_positions(ctx, orc):
    import torch

    rng = np.random.default_rng(3)
    kvw, n_ctx = 256, 40
    k = (rng.standard_normal((5, kvw)) * 100).astype(np.float32)
    v = rng.standard_normal((5, kvw)).astype(np.float32)
    kc = torch.zeros((n_ctx, kvw), dtype=torch.int16).cuda()
    vc = torch.zeros_like(kc)
    ctx.kv_store(dev(k), dev(v), kvw, 10, n_ctx, kc, vc)
    pos = torch.tensor([30], dtype=torch.int32).cuda()
    ctx.kv_store(dev(k[:2]), dev(v[:2]), kvw, 0, n_ctx, kc, vc, pos_dev=pos)
    K, V = host(kc).view(np.uint16), host(vc).view(np.uint16)
    assert np.array_equal(K[10:15], orc.f16_store(k)) and np.array_equal(V[10:15], orc.f16_store(v))
    assert np.array_equal(K[30:32], orc.f16_store(k[:2]))
    assert not K[:10].any() and not K[15:30].any() and not K[32:].any()
    from kestrel_amd.kmoe import KmoeError

    with pytest.raises(KmoeError):  # EngineError::ContextFull (transformer.rs:280-282)
        ctx.kv_store(dev(k), dev(v), kvw, 36, n_ctx, kc, vc)


@pytest.mark.parametrize("nh,nkv,hd,S,pos0", [(8, 8, 64, 1, 0), (8, 2, 64, 1, 63), (8, 2, 128, 1, 64),
                                              (32, 8, 128, 1, 200), (16, 4, 128, 37, 0), (4, 1, 64, 20, 50),
                                              (16, 2, 128, 1, 1023)])
def test_attention(ctx, orc, nh, nkv, hd, S, pos0):
    import torch

    rng = np.random.default_rng(nh + S + pos0)
    n_ctx = 1024
    kvw = nkv * hd
    kc = orc.f16_store(rng.standard_normal((n_ctx, kvw)) * 2)
    vc = orc.f16_store(rng.standard_normal((n_ctx, kvw)))
    q = rng.standard_normal((S, nh * hd)).astype(np.float32)
    ref = orc.attention(q, kc, vc, nh, nkv, hd, pos0)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    got = host(ctx.attention(dev(q), kd, vd, nh, nkv, hd, pos0, n_ctx))
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    pos = torch.tensor([pos0], dtype=torch.int32).cuda()
    got2 = host(ctx.attention(dev(q), kd, vd, nh, nkv, hd, 0, n_ctx, pos_dev=pos))
    assert np.abs(got2 - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("t,rows,cols,S,regime", [(Q4_K, 3072, 2048, 1, 0), (Q8_0, 768, 256, 2, 0),
                                                  (Q6_K, 1000, 512, 1, 1), (Q4_K, 512, 1024, 5, 0),
                                                  (Q4_K, 256, 768, 3, 2)])
def test_norm_matmul_is_rmsnorm_then_matmul(ctx, orc, t, rows, cols, S, regime):
    """The fused norm (+ int8 rows for the integer path) gives the same bits
    as kmoe_rmsnorm followed by kmoe_matmul, on every path."""
    rng = np.random.default_rng(rows + S)
    w = random_blocks(t, rows, cols, seed=rows)
    x = rng.standard_normal((S, cols)).astype(np.float32)
    y = rng.standard_normal((S, cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    ctx.set_regime(regime)
    try:
        x1, x2 = dev(x), dev(x)
        got = host(ctx.norm_matmul(x1, dev(nw), 1e-5, t, dev(w), rows, cols, y=dev(y)))
        h = ctx.rmsnorm(x2, dev(nw), 1e-5, y=dev(y))
        ref = host(ctx.matmul(t, dev(w), rows, cols, h))
    finally:
        ctx.set_regime(0)
    assert np.array_equal(host(x1), host(x2))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("neox", [True, False])
def test_rope_kv_store_is_rope_then_store(ctx, orc, neox):
    import torch

    rng = np.random.default_rng(11)
    S, nh, nkv, hd, rd, n_ctx = 3, 8, 2, 128, 64, 64
    q = rng.standard_normal((S, nh * hd)).astype(np.float32)
    k = rng.standard_normal((S, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((S, nkv * hd)).astype(np.float32)
    f = orc.rope_inv_freq(10000.0, rd)
    kc = torch.zeros((n_ctx, nkv * hd), dtype=torch.int16).cuda()
    vc = torch.zeros_like(kc)
    pos = torch.tensor([20], dtype=torch.int32).cuda()
    qo = host(ctx.rope_kv_store(dev(q), dev(k), dev(v), nh, nkv, hd, rd, 1, dev(f), neox, n_ctx, kc, vc, pos_dev=pos))
    # the same bits as kmoe_rope + kmoe_kv_store; the oracle within rounding of sin/cos
    q_ref = host(ctx.rope(dev(q), nh, hd, rd, 21, dev(f), neox))
    k_ref = host(ctx.rope(dev(k), nkv, hd, rd, 21, dev(f), neox))
    assert np.array_equal(qo, q_ref)
    ro = orc.rope(q, nh, hd, rd, 21, f, neox)
    assert np.abs(qo - ro).max() <= 2e-6 * np.abs(ro).max()
    K, V = host(kc).view(np.uint16), host(vc).view(np.uint16)
    assert np.array_equal(K[21:24], orc.f16_store(k_ref))
    assert np.array_equal(V[21:24], orc.f16_store(v))
    assert not K[:21].any() and not K[24:].any()


@pytest.mark.parametrize("t,S,pos0,regime", [(Q4_K, 1, 10, 0), (Q4_K, 1, 300, 0), (Q8_0, 2, 70, 0), (Q6_K, 1, 5, 1),
                                             (Q4_K, 5, 0, 0), (Q4_K, 1, 130, 2), (Q8_0, 1, 200, 0),
                                             (Q8_0, 1, 520, 1)])
def test_attention_matmul_is_attention_then_matmul(ctx, orc, t, S, pos0, regime):
    """The int8 rows written by the attention kernel feed the projection with
    the same bits as kmoe_attention followed by kmoe_matmul, with one chunk or
    several (the merged path), on every regime's path."""
    rng = np.random.default_rng(pos0 + S)
    nh, nkv, hd, n_ctx, rows = 16, 4, 128, 1024, 512
    kc = orc.f16_store(rng.standard_normal((n_ctx, nkv * hd)))
    vc = orc.f16_store(rng.standard_normal((n_ctx, nkv * hd)))
    q = rng.standard_normal((S, nh * hd)).astype(np.float32)
    w = random_blocks(t, rows, nh * hd, seed=5)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    ctx.set_regime(regime)
    try:
        got = host(ctx.attention_matmul(dev(q), kd, vd, nh, nkv, hd, pos0, n_ctx, t, dev(w), rows))
        a = ctx.attention(dev(q), kd, vd, nh, nkv, hd, pos0, n_ctx)
        ref = host(ctx.matmul(t, dev(w), rows, nh * hd, a))
    finally:
        ctx.set_regime(0)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("nh,nkv,hd,S,pos0", [(16, 16, 128, 12, 250), (16, 4, 128, 6, 60), (8, 2, 64, 5, 508),
                                              (4, 1, 128, 3, 700), (16, 16, 128, 2, 0)])
def test_attention_one_row_is_row_of_batch(ctx, orc, nh, nkv, hd, S, pos0):
    """One query row per call (a work-group per head, the chunks over its
    waves, merged in LDS up to 512 positions and across work-groups beyond)
    gives the bits of the same row in a batch call (a work-group per chunk),
    twice in a row: the handoff counters are zero again after each call."""
    rng = np.random.default_rng(nh + S + pos0)
    n_ctx = 1024
    kvw = nkv * hd
    kc = orc.f16_store(rng.standard_normal((n_ctx, kvw)) * 2)
    vc = orc.f16_store(rng.standard_normal((n_ctx, kvw)))
    q = rng.standard_normal((S, nh * hd)).astype(np.float32)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    batch = host(ctx.attention(dev(q), kd, vd, nh, nkv, hd, pos0, n_ctx))
    for _ in range(2):
        for s in range(S):
            one = host(ctx.attention(dev(q[s:s + 1]), kd, vd, nh, nkv, hd, pos0 + s, n_ctx))
            assert np.array_equal(one.view(np.uint32), batch[s:s + 1].view(np.uint32)), s
    ref = orc.attention(q, kc, vc, nh, nkv, hd, pos0)
    assert np.abs(batch - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_attention_prefill_past_one_super_chunk_twice(ctx, orc):
    """300 prompt rows (later rows span two 256-position super-chunks and merge
    across work-groups), run twice: the handoff counters are zero again after
    every call."""
    rng = np.random.default_rng(12)
    nh, nkv, hd, S, n_ctx = 8, 2, 128, 300, 512
    kc = orc.f16_store(rng.standard_normal((n_ctx, nkv * hd)))
    vc = orc.f16_store(rng.standard_normal((n_ctx, nkv * hd)))
    q = rng.standard_normal((S, nh * hd)).astype(np.float32)
    ref = orc.attention(q, kc, vc, nh, nkv, hd, 0)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    for _ in range(2):
        got = host(ctx.attention(dev(q), kd, vd, nh, nkv, hd, 0, n_ctx))
        assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_swiglu_add_rows_argmax(ctx, orc):
    rng = np.random.default_rng(9)
    g = (rng.standard_normal(5000) * 4).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    got = host(ctx.swiglu(dev(g), dev(u)))
    ref = orc.swiglu(g, u)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    x = rng.standard_normal((3, 40)).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    assert np.array_equal(host(ctx.add_rows(dev(x), dev(b))), x + b)
    for l in (np.array([1, 3, 3, 2], np.float32), np.array([0, np.nan, 5, 5], np.float32),
              np.array([np.nan, 1, 2], np.float32), rng.standard_normal(151936).astype(np.float32),
              np.full(70000, -1.0, np.float32)):
        assert int(host(ctx.argmax(dev(l)))[0]) == orc.argmax(l)
    # the vocabulary's length and ragged ones: the largest value in the last
    # whole 16-byte piece, in the values past it, tied across threads, NaN first
    for n, at in ((102400, 102399), (102403, 102402), (102403, 102399), (70001, 3), (5, 4)):
        l = rng.standard_normal(n).astype(np.float32)
        l[at] = 9.0
        assert int(host(ctx.argmax(dev(l)))[0]) == orc.argmax(l) == at
    l = rng.standard_normal(102400).astype(np.float32)
    l[[4097, 60000, 4096 * 3 + 1]] = 7.0
    l[0] = np.nan
    assert int(host(ctx.argmax(dev(l)))[0]) == orc.argmax(l) == 0
    l[0] = 0.0
    assert int(host(ctx.argmax(dev(l)))[0]) == orc.argmax(l) == 4097
    # an unaligned start (a row of a larger buffer)
    big = dev(rng.standard_normal(1 + 102400).astype(np.float32))
    assert int(host(ctx.argmax(big[1:]))[0]) == orc.argmax(host(big[1:]))


MODELS = {
    "llama_dense": dict(arch="llama", n_layer=2, d=256, nh=4, nkv=2, hd=64, ff=512, vocab=1000),
    "llama_dense_tied_q8": dict(arch="llama", n_layer=2, d=256, nh=4, nkv=4, hd=64, ff=512, vocab=700,
                                wtype=Q8_0, head_type=None, embed_type=Q4_K, rope_dim=32),
    "qwen3moe": dict(arch="qwen3moe", n_layer=2, d=512, nh=8, nkv=2, hd=64, ff=256, vocab=900, qk_norm=True,
                     moe=dict(n_expert=8, n_expert_used=2, types=(Q4_K, Q4_K, Q6_K))),
    "qwen2moe_shared_bias": dict(arch="qwen2moe", n_layer=2, d=256, nh=4, nkv=2, hd=64, ff=256, vocab=800,
                                 bias=True, shared_ff=512, moe=dict(n_expert=8, n_expert_used=4)),
    "mixtral_like_hd128": dict(arch="llama", n_layer=2, d=512, nh=4, nkv=2, hd=128, ff=512, vocab=600,
                               moe=dict(n_expert=4, n_expert_used=2), n_batch=4),
}


@pytest.mark.parametrize("regime", [2, 0])
@pytest.mark.parametrize("name", list(MODELS))
def test_decoder_forward_matches_oracle(ctx, orc, name, regime):
    """Prompt (chunked by n_batch where set), then single-token steps, the
    last row's logits compared with the oracle's Transformer at every call.

    Exact regime (f32 activations everywhere, KESTREL_EXACT): within 1e-3
    relative L2 and 2e-3 of the logit scale (the reference's bound against
    llama.cpp in that mode, tests/oracle.rs:75-77, 115). AVX2 regime (int8
    activations below 4 rows, the reference host's default): an f32
    difference of 1e-7 can flip one int8 rounding, which moves an output by
    1/127 of its block's largest value, so the bound is the reference's own
    for its int8 path, 6e-2 of the logit scale (tests/oracle.rs:124-126)."""
    from kestrel_amd.decoder import Decoder

    hp, T = decoder_model(seed=list(MODELS).index(name) + 1, **MODELS[name])
    ref = orc.Transformer(hp, T, regime=regime)
    ctx.set_regime(regime)
    dec = Decoder(ctx, hp, T)
    try:
        rng = np.random.default_rng(5)
        prompt = rng.integers(0, T["token_embd.weight"][1][1], 9).tolist()
        steps = [prompt] + [[int(t)] for t in rng.integers(0, T["token_embd.weight"][1][1], 4)]
        for toks in steps:
            a = host(dec.forward(toks))
            b = ref.forward(toks)
            scale = max(1.0, float(np.abs(b).max()))
            md = float(np.abs(a - b).max())
            if regime == 2:
                assert rel_l2(a, b) < 1e-3 and md <= 2e-3 * scale, (name, len(toks), rel_l2(a, b), md, scale)
            else:
                assert md <= 6e-2 * scale, (name, len(toks), md, scale)
        assert dec.cached == ref.cached == 13
    finally:
        ctx.set_regime(0)
        dec.close()


@pytest.mark.parametrize("regime", [2, 0, 1])
@pytest.mark.parametrize("name", ["llama_dense", "qwen3moe"])
def test_greedy_decode_graph_matches_eager_and_oracle(ctx, orc, name, regime):
    """Greedy decoding (sampler.rs:58-59) with the step captured once as a
    HIP graph and replayed: the same tokens as eager steps in every regime
    (the AVX2 and int8 regimes run the single-token fast paths under replay:
    RoPE and the KV store in the projection's epilogue from the device
    position, the FFN norm inside the router kernel, the selection inside
    gate/up). Against the oracle's argmax over its own logits fed back step by
    step, up to the first step whose top two logits are closer than the
    numeric deviation between the two (4 x the largest logit difference
    measured on the prompt, at least 1e-3 of the logit scale): a near-tie may
    part the sequences legitimately."""
    from kestrel_amd.decoder import Decoder

    hp, T = decoder_model(seed=7, **MODELS[name])
    prompt = [5, 17, 99, 3]
    outs = []
    ctx.set_regime(regime)
    try:
        for use_graph in (True, False):
            dec = Decoder(ctx, hp, T)
            try:
                logits = host(dec.forward(prompt))
                first = int(np.argmax(logits))
                toks = host(dec.decode_greedy(first, 12, use_graph=use_graph)).tolist()
                outs.append([first] + toks)
                prompt_logits = logits
            finally:
                dec.close()
    finally:
        ctx.set_regime(0)
    assert outs[0] == outs[1]
    ref = orc.Transformer(hp, T, regime=regime)
    l = ref.forward(prompt)
    dev_abs = float(np.abs(prompt_logits - l).max())
    seq = []
    for i in range(13):
        top = np.sort(l)[-2:]
        if top[1] - top[0] < max(4.0 * dev_abs, 1e-3 * max(1.0, float(np.abs(l).max()))):
            break
        seq.append(orc.argmax(l))
        l = ref.forward([seq[-1]])
    assert len(seq) >= 2 and outs[0][:len(seq)] == seq, (seq, outs[0], dev_abs)


@pytest.mark.parametrize("regime", [2, 0])
def test_dsv2lite_stack_reduced_depth_matches_oracle(ctx, orc, regime):
    """The DeepSeek-V2-Lite-shaped stack at its own dimensions, three of its
    27 layers: layer 0 dense (FFN 10944, Q8_0 down), then two MoE layers (64
    routed experts of FFN 1408, top-6, unrenormalised weights, Q8_0 down,
    plus the ungated 2816 shared FFN with a Q6_K down); 16 heads x 128 MHA;
    vocab 102400 with a Q4_K embedding and a Q6_K head; every layer its own
    weights. A 7-token prompt, then single-token steps fed with the oracle's
    argmax, each call's logits against the oracle's Transformer.

    Exact regime: within 1e-3 relative L2 and 2e-3 of the logit scale (the
    reference's bound in that mode, tests/oracle.rs:75-77, 115). AVX2 regime
    (the reference host's default: int8 activations below 4 rows): an f32
    difference of one ulp can flip an int8 rounding, which moves one element
    of a row by 1/127 of its block's largest value, and the layers carry such
    moves forward; the oracle's own logits move by about 1.5% relative L2
    when 64 of layer 0's attention-norm weights are nudged by one ulp. So a
    second oracle with exactly that nudge, fed the same tokens, measures the
    spread per call, and the GPU must stay within 3 x that spread of the
    oracle; and it must give the oracle's argmax at every call whose top two
    logits are further apart than 4 x the largest logit difference measured
    on the prompt (at least 1e-3 of the logit scale), at least two calls
    being that decisive."""
    from kestrel_amd.decoder import Decoder

    rng = np.random.default_rng(23)
    hp, T = stack_model(DSV2LITE, rng, n_ctx=32, n_layer=3, share=False)
    V = DSV2LITE["vocab"]
    ref = orc.Transformer(hp, T, regime=regime)
    nudged = None
    if regime != 2:
        ty, dims, b = T["blk.0.attn_norm.weight"]
        w = b.view(np.float32).copy()
        at = np.random.default_rng(100).choice(w.size, 64, replace=False)
        w[at] = np.nextafter(w[at], np.float32(2))
        nudged = orc.Transformer(hp, {**T, "blk.0.attn_norm.weight": (ty, dims, w.view(np.uint8))}, regime=regime)
    ctx.set_regime(regime)
    dec = Decoder(ctx, hp, T)
    try:
        prompt = rng.integers(0, V, 7).tolist()
        toks = prompt
        a, b = host(dec.forward(toks)), ref.forward(toks)
        dev_abs = float(np.abs(a - b).max())
        decisive, errs, spreads = 0, [], []
        for i in range(6):
            scale = max(1.0, float(np.abs(b).max()))
            err = rel_l2(a, b)
            errs.append(err)
            assert np.isfinite(a).all()
            if regime == 2:
                assert err < 1e-3 and float(np.abs(a - b).max()) <= 2e-3 * scale, (i, err, scale)
            else:
                spread = rel_l2(nudged.forward(toks), b)
                spreads.append(spread)
                assert err <= 3.0 * spread, (i, err, spread)
            top = np.sort(b)[-2:]
            if top[1] - top[0] >= max(4.0 * dev_abs, 1e-3 * scale):
                assert orc.argmax(a) == orc.argmax(b), (i, dev_abs, err)
                decisive += 1
            toks = [orc.argmax(b)]
            a, b = host(dec.forward(toks)), ref.forward(toks)
        assert decisive >= 2, decisive
        print(f"regime {regime}: {decisive} decisive argmax of 6, prompt max |diff| {dev_abs:.3e}, "
              f"rel L2 {' '.join(f'{e:.2e}' for e in errs)}, oracle spread {' '.join(f'{e:.2e}' for e in spreads)}")
    finally:
        ctx.set_regime(0)
        dec.close()


def test_dsv2lite_stack_full_depth_greedy_graph_equals_eager(ctx):
    """All 27 layers of the DeepSeek-V2-Lite-shaped stack (attention, expert
    and dense bytes shared between layers on the host, routers per layer):
    after a 16-token prompt, 8 greedy steps replayed as one captured HIP graph
    give the same tokens as the same steps launched eagerly, and as
    single-token forward() calls at host positions, with every logit finite."""
    import torch

    from kestrel_amd.decoder import Decoder

    rng = np.random.default_rng(11)
    hp, T = stack_model(DSV2LITE, rng, n_ctx=48)
    dec = Decoder(ctx, hp, T)
    try:
        prompt = rng.integers(0, DSV2LITE["vocab"], 16).tolist()
        logits = host(dec.forward(prompt))
        assert np.isfinite(logits).all()
        first = int(np.argmax(logits))
        c0 = dec.cached
        tg = host(dec.decode_greedy(first, 8, use_graph=True)).tolist()
        assert bool(torch.isfinite(dec._graph_bufs["logits"]).all())
        dec.cached = c0
        te = host(dec.decode_greedy(first, 8, use_graph=False)).tolist()
        assert tg == te, (tg, te)
        dec.cached = c0
        tok, tf = first, []
        for _ in range(8):
            l = host(dec.forward([tok]))
            assert np.isfinite(l).all()
            tok = int(np.argmax(l))
            tf.append(tok)
        assert tf == tg, (tf, tg)
    finally:
        dec.close()


def test_greedy_graph_recaptured_after_workspace_grows(ctx, orc):
    """forward(4 tokens) -> greedy steps (captured) -> forward(a 48-token
    chunk, which reallocates the context's workspace the graph pointed into)
    -> greedy steps again: the second run must capture anew (the workspace
    generation moved), and every token must equal the eager path's."""
    from kestrel_amd.decoder import Decoder
    from kestrel_amd.kmoe import Context

    hp, T = decoder_model(seed=11, **MODELS["qwen3moe"])
    rng = np.random.default_rng(2)
    chunk = rng.integers(0, T["token_embd.weight"][1][1], 48).tolist()
    runs = []
    for use_graph in (True, False):
        c = Context(0)  # a fresh context: its workspaces start small
        dec = Decoder(c, hp, T)
        try:
            first = int(np.argmax(host(dec.forward([5, 17, 99, 3]))))
            a = host(dec.decode_greedy(first, 6, use_graph=use_graph)).tolist()
            g0 = c.workspace_generation()
            first2 = int(np.argmax(host(dec.forward(chunk))))
            grew = c.workspace_generation() != g0
            b = host(dec.decode_greedy(first2, 6, use_graph=use_graph)).tolist()
            runs.append((first, a, first2, b, grew))
        finally:
            dec.close()
            c.sync()
            c.close()
    assert runs[0][4], "the 48-token chunk did not grow the workspace: the test would not exercise a regrow"
    assert runs[0][:4] == runs[1][:4]


def test_decoder_context_full(ctx):
    from kestrel_amd.decoder import Decoder

    hp, T = decoder_model(n_ctx=8, seed=3, **{k: v for k, v in MODELS["llama_dense"].items()})
    dec = Decoder(ctx, hp, T)
    try:
        dec.forward([1, 2, 3, 4, 5])
        with pytest.raises(ValueError):
            dec.forward([1, 2, 3, 4])
    finally:
        dec.close()


@pytest.mark.parametrize("t,cols,nh,nkv,hd,rd,neox,regime,use_dev,fused", [
    (Q4_K, 2048, 16, 4, 128, 128, False, 0, False, True),  # 32 lanes per row: the projection applies RoPE
    (Q4_K, 1024, 8, 2, 64, 32, False, 1, True, True),      # 16 lanes per row, partial rope_dim, device position
    (Q8_0, 2048, 16, 4, 128, 128, False, 0, True, False),  # Q8_0 at 2048 columns: 64 lanes per row
    (Q8_0, 1024, 16, 4, 128, 128, False, 0, True, True),
    (Q4_K, 4096, 8, 2, 128, 128, False, 0, False, False),  # 64 lanes per row: separate kernels
    (Q4_K, 2048, 16, 4, 128, 128, True, 0, False, True),   # neox pairs over the whole head
    (Q4_K, 1024, 8, 2, 64, 64, True, 1, True, True),       # neox, 16 lanes per row, device position
    (Q8_0, 1024, 16, 4, 128, 128, True, 0, True, True),
    (Q4_K, 1024, 8, 2, 64, 32, True, 0, False, False),     # neox over part of the head: separate kernels
    (Q4_K, 2048, 16, 4, 128, 128, False, 2, False, False),  # exact regime: separate kernels
])
@pytest.mark.parametrize("out_of_place", [False, True])
def test_norm_matmul_rope_kv_is_norm_matmul_then_rope_kv(ctx, orc, t, cols, nh, nkv, hd, rd, neox, regime, use_dev,
                                                         fused, out_of_place):
    """kmoe_norm_matmul_rope_kv against kmoe_norm_matmul followed by
    kmoe_rope_kv_store on one token: the residual (in place, or into x_out
    with x untouched), the normed row, the projection, the rotated q and both
    caches are the same bits, for two positions in a row (with and without
    the residual add); the RoPE epilogue ran in the projection where the
    geometry allows it, and with x_out on K-quant rows so did the norm (one
    kernel)."""
    import torch

    rows, n_ctx = (nh + 2 * nkv) * hd, 16
    nq, kvw = nh * hd, nkv * hd
    rng = np.random.default_rng(cols + rd)
    w = dev(random_blocks(t, rows, cols, seed=cols))
    nw = dev((1 + 0.1 * rng.standard_normal(cols)).astype(np.float32))
    f = dev(orc.rope_inv_freq(10000.0, rd))
    caches = [torch.zeros((n_ctx, kvw), dtype=torch.int16).cuda() for _ in range(4)]
    ctx.set_regime(regime)
    try:
        for pos in (5, 6):
            x = rng.standard_normal((1, cols)).astype(np.float32)
            # the second position without the residual add
            y = dev(rng.standard_normal((1, cols)).astype(np.float32)) if pos == 5 else None
            xa, xb = dev(x), dev(x)
            pos_dev = torch.tensor([pos - 2], dtype=torch.int32).cuda() if use_dev else None
            p0 = 2 if use_dev else pos
            ha = torch.empty((1, cols), dtype=torch.float32).cuda()
            qkva = torch.empty((1, rows), dtype=torch.float32).cuda()
            xo = torch.full((1, cols), float("nan"), dtype=torch.float32).cuda() if out_of_place else None
            ctx.profile_enable(True)
            qa = ctx.norm_matmul_rope_kv(xa, nw, 1e-5, t, w, cols, nh, nkv, hd, rd, p0, f, neox, n_ctx, caches[0],
                                         caches[1], y=y, pos_dev=pos_dev, h=ha, qkv=qkva, x_out=xo)
            assert ctx.profile_read("matvec_qkv_rope")[1] == (1 if fused else 0)
            one_kernel = fused and out_of_place and t != Q8_0
            if one_kernel:
                assert ctx.profile_read("rmsnorm_quant")[1] == 0
            ctx.profile_enable(False)
            if out_of_place:
                assert np.array_equal(host(xa).view(np.uint32), x.view(np.uint32))
                xa = xo
            hb = torch.empty((1, cols), dtype=torch.float32).cuda()
            qkvb = ctx.norm_matmul(xb, nw, 1e-5, t, w, rows, cols, y=y, h=hb)
            qb = ctx.rope_kv_store(qkvb[:, :nq], qkvb[:, nq:nq + kvw], qkvb[:, nq + kvw:], nh, nkv, hd, rd, p0, f,
                                   neox, n_ctx, caches[2], caches[3], pos_dev)
            for u, v in ((xa, xb), (ha, hb), (qkva, qkvb), (qa, qb)):
                assert np.array_equal(host(u).view(np.uint32), host(v).view(np.uint32)), pos
            for u, v in ((caches[0], caches[2]), (caches[1], caches[3])):
                assert np.array_equal(host(u), host(v)), pos
            assert host(caches[0])[pos].any() and host(caches[1])[pos].any()
    finally:
        ctx.profile_enable(False)
        ctx.set_regime(0)


def test_norm_matmul_rope_kv_rejects_bad_arguments(ctx, orc):
    """The one-token projection + RoPE entry point reports the errors of the
    two calls it stands for: odd or oversized rope_dim, a full context at a
    host position, a missing cache; nothing is written to the caches."""
    import torch

    from kestrel_amd.kmoe import KmoeError

    nh, nkv, hd, cols, n_ctx = 4, 2, 64, 256, 8
    rows = (nh + 2 * nkv) * hd
    w = dev(random_blocks(Q4_K, rows, cols, seed=3))
    nw = dev(np.ones(cols, np.float32))
    f = dev(orc.rope_inv_freq(10000.0, hd))
    kc = torch.zeros((n_ctx, nkv * hd), dtype=torch.int16).cuda()
    vc = torch.zeros_like(kc)
    x = dev(np.ones((1, cols), np.float32))
    for rd, pos in ((hd - 1, 0), (hd + 2, 0), (hd, n_ctx)):
        with pytest.raises(KmoeError):
            ctx.norm_matmul_rope_kv(x, nw, 1e-5, Q4_K, w, cols, nh, nkv, hd, rd, pos, f, False, n_ctx, kc, vc)
    h = torch.empty((1, cols), dtype=torch.float32).cuda()
    qkv = torch.empty((1, rows), dtype=torch.float32).cuda()
    q_out = torch.empty((1, nh * hd), dtype=torch.float32).cuda()
    rc = ctx.lib.kmoe_norm_matmul_rope_kv(ctx.h, x.data_ptr(), None, nw.data_ptr(), 1e-5, Q4_K, w.data_ptr(),
                                          w.numel(), cols, h.data_ptr(), qkv.data_ptr(), nh, nkv, hd, hd, 0, None,
                                          f.data_ptr(), 0, n_ctx, q_out.data_ptr(), None, vc.data_ptr(), None)
    assert rc != 0
    assert not host(kc).any() and not host(vc).any()


def test_norm_moe_ffn_rejects_null_rows(ctx, orc):
    """kmoe_norm_moe_ffn needs x, the norm weights and f for s_rows > 0."""
    spec = LayerSpec(8, 2, 256, 256, Q4_K, seed=9)
    lid = 900
    spec.upload(ctx, lid)
    try:
        x = dev(np.ones((1, 256), np.float32))
        out = dev(np.zeros((1, 256), np.float32))
        for args in ((None, x, x), (x, None, x), (x, x, None)):
            p = [a.data_ptr() if a is not None else None for a in args]
            rc = ctx.lib.kmoe_norm_moe_ffn(ctx.h, lid, p[0], None, p[1], 1e-5, 1, p[2], out.data_ptr())
            assert rc != 0
        assert not host(out).any()
    finally:
        ctx.layer_destroy(lid)
