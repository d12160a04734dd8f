"""Committed golden fixtures (tests/golden/, written by make_golden.py from the
oracle): the CPU tests pin the oracle and its input generators against them
bit for bit; the GPU tests hold the HIP path to them at the parity bar
(routing, permutation and integer accumulators exact, fp32 within 1e-3
relative L2)."""
import json
import os

import numpy as np
import pytest

from tests.golden import make_golden as mg
from tests.helpers import Q4_K, rel_l2

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name)) as z:  # allow_pickle=False
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def manifest():
    with open(os.path.join(HERE, "manifest.json")) as f:
        return json.load(f)


def test_generators_reproduce_the_fixture_inputs(manifest):
    spec, h = mg.c1_inputs()
    w2, x2 = mg.c2_inputs()
    assert mg.input_hashes(spec, h, w2, x2) == manifest["inputs_sha256"]


def test_oracle_reproduces_c1(manifest):
    spec, h = mg.c1_inputs()
    got = mg.c1_outputs(spec, h)
    ref = load("c1_q8_0_moe.npz")
    for k in ref:
        assert np.array_equal(got[k], ref[k]), k
        assert mg.sha(got[k]) == manifest["outputs_sha256"][f"c1.{k}"], k


def test_oracle_reproduces_c2(manifest):
    got = mg.c2_outputs(*mg.c2_inputs())
    ref = load("c2_q4k_rows.npz")
    for k in ref:
        assert np.array_equal(got[k], ref[k]), k
        assert mg.sha(got[k]) == manifest["outputs_sha256"][f"c2.{k}"], k


def test_fixture_c1_invariants():
    """Checks that do not go through the oracle: the permutation is the stable
    sort of the flat slots by expert (transformer.rs:525-535) and the offsets
    are its run starts; renormalised weights sum to one."""
    r = load("c1_q8_0_moe.npz")
    flat = r["idx"].reshape(-1)
    assert np.array_equal(r["perm"], np.argsort(flat, kind="stable"))
    assert np.array_equal(r["offsets"], np.searchsorted(np.sort(flat), np.arange(9)))
    assert np.allclose(r["w"].sum(axis=1), 1.0, atol=1e-6)


# ------------------------------------------------------------------- GPU side
@pytest.fixture(scope="module")
def ctx():
    import torch

    from kestrel_amd.kmoe import Context

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    c = Context(0)
    yield c
    c.sync()
    c.close()


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.gpu
def test_gpu_c1_matches_golden(ctx):
    spec, h = mg.c1_inputs()
    ref = load("c1_q8_0_moe.npz")
    spec.upload(ctx, 300)
    try:
        out = _host(ctx.moe_ffn(300, _dev(h)))
        idx, w, perm, off = (_host(t) for t in ctx.last_routing(16, 2, 8))
    finally:
        ctx.layer_destroy(300)
    assert np.array_equal(idx.view(np.uint32), ref["idx"])
    assert np.allclose(w, ref["w"], rtol=1e-6, atol=0)
    assert np.array_equal(perm.view(np.uint32), ref["perm"])
    assert np.array_equal(off.view(np.uint32), ref["offsets"])
    assert rel_l2(out, ref["out"]) < 1e-3


@pytest.mark.gpu
def test_gpu_c2_rows_match_golden(ctx):
    w, x = mg.c2_inputs()
    ref = load("c2_q4k_rows.npz")
    xq, xd, xs = (_host(t) for t in ctx.quantize_q8k(_dev(x)))
    assert np.array_equal(xq.reshape(ref["xq"].shape), ref["xq"])
    assert np.array_equal(xd.reshape(ref["xd"].shape), ref["xd"])
    assert np.array_equal(xs.reshape(ref["bsums"].shape), ref["bsums"])
    sumi, mins = (_host(t) for t in ctx.q4k_block_sums(_dev(w), 8, 4096, _dev(ref["xq"]), _dev(ref["bsums"])))
    assert np.array_equal(sumi.reshape(ref["sumi"].shape), ref["sumi"])
    assert np.array_equal(mins.reshape(ref["mins"].shape), ref["mins"])
    ctx.set_regime(1)
    try:
        y = _host(ctx.matmul(Q4_K, _dev(w), 8, 4096, _dev(x)))
    finally:
        ctx.set_regime(0)
    assert rel_l2(y.reshape(-1), ref["y"].reshape(-1)) < 1e-3
