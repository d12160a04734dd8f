"""kmoe_measure: the GPU figures kestrel's planner takes from a table of known
parts today (kestrel-hw gpu.rs:28-34, planner cost.rs:26-83, :102), measured."""
import pytest

pytestmark = pytest.mark.gpu


def test_measurements_are_physical():
    import torch

    from kestrel_amd.kmoe import Context

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    c = Context(0)
    try:
        before = c.vram_usage()[0]
        m = c.measure()
        # the 250 MB measurement buffer is released; only the context's
        # persistent workspace may have grown (the GEMV's activation rows)
        assert c.vram_usage()[0] - before < 16 << 20
        assert m["vram_total"] > 64 << 30 and 0 < m["vram_free"] <= m["vram_total"]
        # read + written bytes of a device copy: below twice the 8 TB/s HBM peak
        assert 1e12 < m["hbm_copy_bps"] < 1.7e13, m
        for t, v in m["gemv_bps"].items():
            assert 3e11 < v < 8.5e12, (t, m)  # weight bytes of a decode GEMV: below the HBM peak
        assert 1e9 < m["h2d_bps"] < 1.5e11 and 1e9 < m["d2h_bps"] < 1.5e11, m
        assert 1e-7 < m["launch_s"] < 1e-4, m
        print(m)
    finally:
        c.sync()
        c.close()
