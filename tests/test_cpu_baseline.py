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


def test_bench_reads_every_kernel_from_the_committed_profile():
    """bench.py's roofline takes each kernel's HBM traffic from the committed
    rocprofv3 summary of the headline workload and its algorithmic bytes from
    the byte model: both must cover every kernel the events time."""
    import bench
    import dpep
    kb = bench.kernel_bytes(1100000, 2048, 2048, 4)
    keys = [k for k in dpep.KERNEL_KEYS if k != "step"]
    # bin_fill_fresh: the counted K3 of two-pass steps, timed in the bin_fill slot
    assert set(kb) == set(keys) == set(bench.PMC_NAMES) - {"bin_fill_fresh"}
    for k in keys + ["bin_fill_fresh"]:
        t = bench.pmc_traffic(k)
        a = kb["bin_fill" if k == "bin_fill_fresh" else k]
        assert t is not None and t >= 0.9 * a, k   # HBM traffic covers the algorithmic bytes
    # one row each: the one-pass K3's own traffic, not a sum over variants
    assert bench.pmc_traffic("bin_fill") < bench.pmc_traffic("bin_fill_fresh")
    # the step's byte model: 40 Nc + 52 MN at float32 with the potential
    assert bench.step_bytes(1100000, 2048, 2048, 4) == 40 * 1100000 + 52 * 2048 * 2048
