"""kmoe_moe_ffn_noalloc (the entry point that allocates nothing) against
kmoe_moe_ffn, through the C ABI: two calls in a row, the second with fewer
tokens, each with the same routing, dispatch and output bits as the existing
entry point and within the oracle's tolerance; no workspace growth and no
VRAM reservation on a fresh context; a size past the static scratch refused."""
import numpy as np
import pytest

from tests.helpers import Q4_K, Q6_K, LayerSpec, rel_l2

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_noalloc_matches_moe_ffn_on_two_calls(orc):
    import torch

    from kestrel_amd.kmoe import Context

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = Context(0)  # fresh: its own workspace starts empty
    spec = LayerSpec(8, 2, 4096, 8192, Q4_K, seed=17, quantized=False, down_type=Q6_K)
    spec.upload(ctx, 0)
    try:
        gen0 = ctx.workspace_generation()
        reserved0 = ctx.vram_usage()[0]
        outs = {}
        for S in (6, 1):  # the second call smaller
            h = orc.normal(900 + S, S * 4096).reshape(S, 4096)
            hd = _dev(h)
            o = torch.full((S, 4096), float("nan"), dtype=torch.float32, device="cuda")
            ctx.check(ctx.lib.kmoe_moe_ffn_noalloc(ctx.h, 0, hd.data_ptr(), S, o.data_ptr()))
            a = _host(o)
            ra = [_host(t) for t in ctx.last_routing(S, spec.k, spec.n_expert)]
            assert ctx.workspace_generation() == gen0 and ctx.vram_usage()[0] == reserved0, "noalloc allocated"
            outs[S] = (h, a, ra)
        for S, (h, a, ra) in outs.items():
            b = _host(ctx.moe_ffn(0, _dev(h)))
            rb = [_host(t) for t in ctx.last_routing(S, spec.k, spec.n_expert)]
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), S
            for x, y in zip(ra, rb):
                assert np.array_equal(x, y), S
            L = spec.oracle_layer()
            ridx, _ = L.route(h)
            assert np.array_equal(ra[0].view(np.uint32), ridx)
            assert rel_l2(a, L.moe_ffn(h)) < 1e-3
        # 4096 tokens need more than the static scratch: refused, nothing run
        from kestrel_amd.kmoe import KmoeError

        big = torch.zeros((4096, 4096), dtype=torch.float32, device="cuda")
        with pytest.raises(KmoeError) as e:
            ctx.check(ctx.lib.kmoe_moe_ffn_noalloc(ctx.h, 0, big.data_ptr(), 4096, big.data_ptr()))
        assert e.value.status == -1 and "static scratch" in str(e.value)
    finally:
        ctx.layer_destroy(0)
        ctx.sync()
        ctx.close()
