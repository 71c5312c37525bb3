"""GPU: steps on cells that move between steps, the way DREAMPlace calls the
step -- the one-pass binning plans each step from the previous step's
counts, and records past a region's room go to their strip's overflow list.

Every step must give, bitwise, what a context that counts before it sorts
(DPEP_FLAG_TWO_PASS) gives on the same cells (integer accumulation makes the
density independent of where records land, and each record's partial force
is summed in the same order either way), and the float64 oracle's results
within the step's tolerances (float32: density/potential rel L-inf <= 1e-5,
fields/forces rel L2 <= 1e-4).  dpep_get_binning_stats reports how each step
binned its cells."""
import numpy as np
import pytest

from conftest import rel_l2, rel_linf

pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    for k in ("density", "potential"):
        e = rel_linf(out[k], ref[k])
        assert e <= 1e-5, f"{tag} {k} rel Linf {e:.3e}"
    for k in ("field_x", "field_y", "grad_x", "grad_y"):
        e = rel_l2(out[k], ref[k])
        assert e <= 1e-4, f"{tag} {k} rel L2 {e:.3e}"


def _contexts(w, dtype=np.float32):
    import dpep
    one = dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype)
    two = dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype, two_pass=True)
    for c in (one, two):
        c.set_initial_density(w.d0n.astype(dtype))
    return one, two


def test_drift_keeps_the_plan(oracle):
    """The hotspot loop's drift (N(0, 0.5 bin) per cell per step) on a
    1.1M-cell 2048^2 placement: after the first (counted) step every step
    sorts in one pass with no overflow, and equals the counted step."""
    from dpep import workloads
    w = workloads.make(3, seed=0)
    sx, sy = w.sx, w.sy
    one, two = _contexts(w)
    try:
        for k, px, py in workloads.walk(w, 6):
            print(f"drift step {k}", flush=True)
            a = one.step(px, py, sx, sy)
            st = one.binning_stats()
            b = two.step(px, py, sx, sy)
            assert st["one_pass"] == (1 if k > 0 else 0)
            assert st["overflow_records"] == 0 and st["overflow_runs_max"] == 0
            assert two.binning_stats()["one_pass"] == 0
            assert st["records"] == two.binning_stats()["records"]
            for key in a:
                assert np.array_equal(a[key], b[key]), f"step {k} {key}"
        _check(a, oracle.step(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                              d0n=w.d0n.astype(np.float32)), "drift")
    finally:
        one.close()
        two.close()


def test_respread_overflows_and_matches_counted_steps(oracle):
    """A placement and a uniform placement of the same cells, alternating
    every step: each one-pass step is planned from the other placement, so
    a few percent of its records overflow into per-strip lists.  Every step
    equals the counted step bitwise; two are checked against the oracle."""
    from dpep import workloads
    w = workloads.small(3, seed=41, cells=300000, grid=1024)
    pa, pb_, sx, sy = w.cells(np.float32)
    rng = np.random.default_rng(42)
    ux = (rng.uniform(0, 1, w.nc) * (w.xh - w.xl - sx) + w.xl).astype(np.float32)
    uy = (rng.uniform(0, 1, w.nc) * (w.yh - w.yl - sy) + w.yl).astype(np.float32)
    one, two = _contexts(w)
    try:
        for k in range(5):
            px, py = (pa, pb_) if k % 2 == 0 else (ux, uy)
            print(f"respread step {k}", flush=True)
            a = one.step(px, py, sx, sy)
            st = one.binning_stats()
            b = two.step(px, py, sx, sy)
            if k > 0:
                assert st["one_pass"] == 1
                assert st["overflow_records"] > 0, st
                assert st["overflow_runs_max"] > 0
            for key in a:
                assert np.array_equal(a[key], b[key]), f"step {k} {key}"
            if k in (1, 4):
                _check(a, oracle.step(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                                      d0n=w.d0n.astype(np.float32)), f"respread {k}")
            print(f"  overflow {st['overflow_records']} of {st['records']} records, "
                  f"at most {st['overflow_runs_max']} runs in a strip", flush=True)
    finally:
        one.close()
        two.close()


def test_overflow_runs_beyond_one_batch(oracle):
    """2.5M cells spread over the die, then all moved into one strip: the
    second step's plan leaves that strip a 64th of the room it needs, so
    every block of cells (more than the 1024 runs K4 and G1 stage in LDS at
    once) adds a run to its overflow list; the walk takes several batches.
    Bitwise equal to a counted step, and the oracle's within tolerance."""
    from dpep import workloads
    n = 2_500_000
    w = workloads.config5(n_mov=n)                    # 512^2, die 27000
    sx, sy = w.sx, w.sy
    rng = np.random.default_rng(43)
    ux = (rng.uniform(0, 1, n) * (w.xh - sx)).astype(np.float32)
    uy = (rng.uniform(0, 1, n) * (w.yh - sy)).astype(np.float32)
    strip = 8 * w.bsx                                 # 8 rows of bins per strip
    x0 = 30 * strip
    bx = (x0 + rng.uniform(0, 1, n) * (strip - sx)).astype(np.float32)
    one, two = _contexts(w)
    try:
        one.step(ux, uy, sx, sy)
        print("band step", flush=True)
        a = one.step(bx, uy, sx, sy)
        st = one.binning_stats()
        b = two.step(bx, uy, sx, sy)
        print(f"  overflow {st['overflow_records']} of {st['records']} records, "
              f"at most {st['overflow_runs_max']} runs in a strip", flush=True)
        assert st["one_pass"] == 1 and st["overflow_runs_max"] > 1024
        for key in a:
            assert np.array_equal(a[key], b[key]), key
        _check(a, oracle.step(bx, uy, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                              d0n=w.d0n.astype(np.float32)), "band")
        # planned from the band's own counts, the next step does not overflow
        one.step(bx, uy, sx, sy)
        assert one.binning_stats()["overflow_records"] == 0
    finally:
        one.close()
        two.close()
