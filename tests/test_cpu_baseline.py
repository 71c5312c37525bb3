"""The float32 OpenMP CPU baseline (timed by bench.py) computes the same step
as the float64 oracle, to float32 accuracy."""
import numpy as np

from conftest import rel_l2, rel_linf


def test_cpu_baseline_matches_oracle(oracle):
    from dpep import workloads
    w = workloads.small(3, seed=2, cells=20000, grid=128)
    px, py, sx, sy = w.cells(np.float32)
    d0 = w.d0n.astype(np.float32)
    cb = oracle.CpuBaseline(w.M, w.N, w.xl, w.yl, w.xh, w.yh)
    got = cb.step(px, py, sx, sy, d0)
    ref = oracle.step(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh, d0n=d0)
    assert rel_linf(got["density"], ref["density"]) < 1e-3
    assert rel_linf(got["potential"], ref["potential"]) < 1e-3
    for k in ("field_x", "field_y", "grad_x", "grad_y"):
        assert rel_l2(got[k], ref[k]) < 1e-3, k
    assert set(got["stage_ms"]) == {"scatter", "solve", "gather"}
    cb.close()
