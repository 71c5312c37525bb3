"""GPU parity: libdpep.so on the MI355X against the float64 oracle, through
the C ABI (ctypes), on the same seeded inputs.

Tolerances (the step's contract):
  float32: density and potential rel L-inf <= 1e-5; field_x/y and per-cell
           forces rel L2 <= 1e-4.
  float64: density and potential rel L-inf <= 1e-10; fields and forces rel
           L2 <= 1e-9 (fixed-point mode: quantum 2^-36 of a bin density).
"""
import ctypes

import numpy as np
import pytest

from conftest import rel_l2, rel_linf

pytestmark = pytest.mark.gpu

TOL = {np.float32: (1e-5, 1e-4), np.float64: (1e-10, 1e-9)}


def check(out, ref, dtype, tag=""):
    tl, tf = TOL[dtype]
    errs = {}
    for k in ("density", "potential"):
        if k in out and k in ref:
            errs[k] = rel_linf(out[k], ref[k])
            assert errs[k] <= tl, f"{tag} {k} rel Linf {errs[k]:.3e} > {tl}"
    for k in ("field_x", "field_y", "grad_x", "grad_y"):
        if k in out and k in ref:
            errs[k] = rel_l2(out[k], ref[k])
            assert errs[k] <= tf, f"{tag} {k} rel L2 {errs[k]:.3e} > {tf}"
    return errs


def run_gpu(w, dtype=np.float32, cells=None, **kw):
    """Two steps on the same cells: the first counts the cells per strip
    before sorting them, the second sorts in one pass into the room the
    first planned.  Both must give bitwise the same outputs; returns the
    second's."""
    import dpep
    px, py, sx, sy = cells if cells is not None else w.cells(dtype)
    with dpep.Context(w.M, w.N, max(len(px), 1), w.xl, w.yl, w.xh, w.yh,
                      dtype=dtype, **kw) as ctx:
        ctx.set_initial_density(w.d0n.astype(dtype))
        first = ctx.step(px, py, sx, sy)
        second = ctx.step(px, py, sx, sy)
    for k in first:
        assert np.array_equal(first[k], second[k], equal_nan=True), \
            f"{k}: the one-pass step differs from the counted one"
    return second


def run_oracle(oracle, w, dtype=np.float32, cells=None, stretch=True):
    px, py, sx, sy = cells if cells is not None else w.cells(dtype)
    return oracle.step(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                       d0n=w.d0n.astype(dtype), stretch=stretch)


# --------------------------------------------------------------------------
# spectral solve alone (no cells; the density is the uploaded D0)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("M,N", [(8, 8), (16, 64), (64, 16), (512, 512),
                                 (2048, 2048), (4096, 4096), (8192, 8), (8, 8192),
                                 (64, 8192)])
def test_solve_random_density(oracle, dtype, M, N):
    import dpep
    if dtype == np.float64 and max(M, N) > 4096:
        pytest.skip("float64 grids are limited to 4096")
    rng = np.random.default_rng(M + 3 * N)
    d0 = rng.random((M, N)).astype(dtype)
    with dpep.Context(M, N, 1, 0.0, 0.0, 70.0, 50.0, dtype=dtype) as ctx:
        ctx.set_initial_density(d0)
        out = ctx.step(*[np.zeros(0, dtype)] * 4)
    phi, fx, fy = oracle.solve(d0.astype(np.float64), 70.0 / M, 50.0 / N)
    check(out, {"density": d0, "potential": phi, "field_x": fx, "field_y": fy},
          dtype, f"{M}x{N}")


@pytest.mark.parametrize("u0,v0", [(3, 5), (0, 1), (1, 0), (31, 17)])
def test_solve_single_mode_closed_form(u0, v0):
    import dpep
    M, N, bsx, bsy = 64, 32, 2.0, 3.0
    t = np.arange(M)[:, None] + 0.5
    s = np.arange(N)[None, :] + 0.5
    rho = np.cos(np.pi * u0 * t / M) * np.cos(np.pi * v0 * s / N)
    with dpep.Context(M, N, 1, 0.0, 0.0, M * bsx, N * bsy, dtype=np.float64) as ctx:
        ctx.set_initial_density(rho)
        out = ctx.step(*[np.zeros(0)] * 4)
    wu = 2 * np.pi * u0 / M
    wv = 2 * np.pi * v0 / N * bsx / bsy
    D = wu * wu + wv * wv
    amp = (2.0 if u0 == 0 else 1.0) * (2.0 if v0 == 0 else 1.0)
    cu, cv = (1.0 if u0 == 0 else 2.0), (1.0 if v0 == 0 else 2.0)
    sx_ = np.sin(np.pi * u0 * t / M) * np.cos(np.pi * v0 * s / N)
    sy_ = np.cos(np.pi * u0 * t / M) * np.sin(np.pi * v0 * s / N)
    np.testing.assert_allclose(out["potential"], amp * cu * cv / D * rho, atol=1e-10)
    np.testing.assert_allclose(out["field_x"], amp * cv * wu / D * sx_, atol=1e-10)
    np.testing.assert_allclose(out["field_y"], amp * cu * wv / D * sy_, atol=1e-10)


# --------------------------------------------------------------------------
# full steps against the oracle
# --------------------------------------------------------------------------
@pytest.mark.parametrize("cfg,cells,grid", [(1, 30000, 128), (2, 30000, 512),
                                            (3, 40000, 256), (5, 60000, 64)])
@pytest.mark.parametrize("det", [False, True])
def test_small_configs(oracle, cfg, cells, grid, det):
    from dpep import workloads
    w = workloads.small(cfg, seed=11, cells=cells, grid=grid)
    check(run_gpu(w, deterministic=det), run_oracle(oracle, w), np.float32,
          f"C{cfg} small det={det}")


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_full_size_configs(oracle, cfg):
    from dpep import workloads
    w = workloads.make(cfg, seed=0)
    errs = check(run_gpu(w), run_oracle(oracle, w), np.float32, f"C{cfg}")
    print(f"C{cfg} full: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))


@pytest.mark.parametrize("n_mov,dtype", [(600_000, np.float32), (1_400_000, np.float32),
                                         (1_800_000, np.float32), (900_000, np.float64)])
def test_one_pass_block_sizes(oracle, n_mov, dtype):
    """The C3 design at cell counts whose one-pass blocks (once_blocks: three
    per CU at float32, two at float64, on a 256-CU MI355X) take 2, 4 and 5
    cells per thread at float32 and 4 at float64 (1.1 M cells, 3 per thread
    at float32 and 5 at float64, and 2.0 M cells, blocks in rounds, are the
    full-size configurations)."""
    from dpep import workloads
    w = workloads.config3(seed=3, n_mov=n_mov)
    errs = check(run_gpu(w, dtype=dtype), run_oracle(oracle, w, dtype=dtype), dtype,
                 f"{n_mov} cells")
    print(f"{n_mov} cells {np.dtype(dtype).name}: " +
          " ".join(f"{k}={v:.2e}" for k, v in errs.items()))


def test_float64_mode(oracle):
    from dpep import workloads
    w = workloads.small(5, seed=3, cells=100000, grid=512)
    for det in (False, True):
        check(run_gpu(w, np.float64, deterministic=det),
              run_oracle(oracle, w, np.float64), np.float64, f"f64 det={det}")


def test_float64_4096_grid(oracle):
    """float64 at 4096 x 4096 (the largest float64 grid): 4-row strips, the
    gather staging two rows of both field maps at a time, the 4096-point
    column and row passes; the C4 recipe with 300 K cells."""
    from dpep import workloads
    w = workloads.small(4, seed=5, cells=300000, grid=4096)
    errs = check(run_gpu(w, np.float64), run_oracle(oracle, w, np.float64), np.float64,
                 "f64 4096")
    print(errs, flush=True)


def test_no_stretch_semantics(oracle):
    """DPEP_FLAG_NO_STRETCH reproduces the TT path's density (original sizes,
    ratio 1: scatter_ttnn_client.py:628-649)."""
    from dpep import workloads
    w = workloads.small(3, seed=4, cells=30000, grid=256)
    check(run_gpu(w, stretch=False), run_oracle(oracle, w, stretch=False),
          np.float32, "no-stretch")


# --------------------------------------------------------------------------
# determinism
# --------------------------------------------------------------------------
def test_deterministic_mode_is_bitwise_reproducible_and_order_free():
    from dpep import workloads
    w = workloads.small(2, seed=5, cells=200000, grid=512)   # hot centre bins
    a = run_gpu(w, deterministic=True)
    b = run_gpu(w, deterministic=True)
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    p = np.random.default_rng(0).permutation(w.nc)
    cells = tuple(np.ascontiguousarray(c[p]) for c in w.cells(np.float32))
    c = run_gpu(w, deterministic=True, cells=cells)
    for k in ("density", "potential", "field_x", "field_y"):
        assert np.array_equal(a[k], c[k]), k


@pytest.mark.parametrize("grid,dtype", [(512, np.float32), (4096, np.float32),
                                        (512, np.float64)])
def test_one_pass_overflow_matches_counted_step(oracle, grid, dtype):
    """A context stepped on one placement, then on a very different one:
    the one-pass sort of the second placement runs out of room in most
    strips (the room was planned for the first), so most of its records go
    to their strips' overflow lists (added into the strip tiles and gathered
    from the staged field rows after the strips' own records).  Its outputs
    must equal, bitwise, those of a context that counts first
    (DPEP_FLAG_TWO_PASS), and the oracle's; a third step (planned from the
    second's counts) overflows no more and gives the same again."""
    import dpep
    from dpep import workloads
    b = workloads.small(5, seed=22, cells=60000, grid=grid)     # one hot square
    cb = b.cells(dtype)
    rng = np.random.default_rng(23)                              # the same cells
    ca = (rng.uniform(b.xl, b.xh - cb[2]).astype(dtype),         # spread out
          rng.uniform(b.yl, b.yh - cb[3]).astype(dtype), cb[2], cb[3])
    with dpep.Context(b.M, b.N, b.nc, b.xl, b.yl, b.xh, b.yh, dtype=dtype) as ctx:
        ctx.set_initial_density(b.d0n.astype(dtype))
        ctx.step(*ca)
        over = ctx.step(*cb)
        st = ctx.binning_stats()
        again = ctx.step(*cb)
        assert ctx.binning_stats()["overflow_records"] == 0
    assert st["one_pass"] == 1 and st["overflow_records"] > st["records"] // 4, st
    with dpep.Context(b.M, b.N, b.nc, b.xl, b.yl, b.xh, b.yh, dtype=dtype,
                      two_pass=True) as ctx:
        ctx.set_initial_density(b.d0n.astype(dtype))
        ref2 = ctx.step(*cb)
    for k in ref2:
        assert np.array_equal(over[k], ref2[k]), f"{k}: overflowing step differs"
        assert np.array_equal(again[k], ref2[k]), f"{k}: re-planned step differs"
    errs = check(over, run_oracle(oracle, b, dtype, cells=cb), dtype,
                 f"overflow {grid} {np.dtype(dtype).name}")
    print(f"one-pass overflow {grid}^2 {np.dtype(dtype).name}: " +
          " ".join(f"{k}={v:.2e}" for k, v in errs.items()))


# --------------------------------------------------------------------------
# edge cases of the boundary
# --------------------------------------------------------------------------
def test_edge_cells(oracle):
    from dpep import workloads
    w = workloads.small(3, seed=6, cells=5000, grid=64)
    px, py, sx, sy = [a.copy() for a in w.cells(np.float32)]
    bs = w.bsx
    # zero / negative sizes, NaN / inf positions, outside the die, wider than
    # the die, exactly on bin edges, straddling the die corner
    px[:12] = [0, 10, np.nan, 100, -5 * w.xh, 2 * w.xh, -3 * bs, 0, 5 * bs, 7 * bs, w.xh - 1, 1]
    py[:12] = [0, 10, 5, np.inf, 10, 10, 5 * bs, 0, 5 * bs, 3 * bs, w.yh - 1, 1]
    sx[:12] = [0, -1, 3, 3, 4, 4, 3 * w.xh, w.xh, bs, 2 * bs, 30, 1e-3]
    sy[:12] = [5, 5, 3, 3, 4, 4, 12, w.yh, bs, 12, 30, 1e-3]
    cells = (px, py, sx, sy)
    out = run_gpu(w, cells=cells)
    ref = run_oracle(oracle, w, cells=cells)
    check(out, ref, np.float32, "edge")
    assert np.all(np.isfinite(out["grad_x"])) and np.all(np.isfinite(out["density"]))
    assert out["grad_x"][0] == 0 and out["grad_x"][1] == 0 and out["grad_x"][2] == 0


@pytest.mark.parametrize("grid", [512, 4096])
def test_tall_cells(oracle, grid):
    """Cells wider than a strip take the side map B: small ones (<= 256 bins)
    are gathered by one thread, larger ones by the whole workgroup, and each
    strip folds only the column blocks its tall cells marked.  Two steps on
    one context: the marks must be cleared by the first."""
    import dpep
    from dpep import workloads
    w = workloads.small(4, seed=12, cells=20000, grid=grid)
    px, py, sx, sy = [a.copy() for a in w.cells(np.float32)]
    rng = np.random.default_rng(12)
    sel = rng.choice(w.nc, w.nc // 10, replace=False)
    sx[sel] = (w.bsx * rng.uniform(4.5, 40.0, sel.size)).astype(np.float32)     # small tall
    big = sel[:8]
    sx[big] = np.float32(300 * w.bsx)                                         # > 256 bins
    sy[big] = np.float32(3 * w.bsy)
    px[sel] = np.minimum(px[sel], np.float32(w.xh - sx[sel]))
    cells = (px, py, sx, sy)
    ref = run_oracle(oracle, w, cells=cells)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh) as ctx:
        ctx.set_initial_density(w.d0n.astype(np.float32))
        first = ctx.step(*cells)
        check(first, ref, np.float32, f"tall {grid} step 1")
        second = ctx.step(*cells)
    for k in first:
        assert np.array_equal(first[k], second[k]), k


def test_no_cells_and_shrinking_cell_count(oracle):
    import dpep
    from dpep import workloads
    w = workloads.small(3, seed=7, cells=20000, grid=128)
    cells = w.cells(np.float32)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh) as ctx:
        ctx.set_initial_density(w.d0n.astype(np.float32))
        out0 = ctx.step(*[np.zeros(0, np.float32)] * 4)
        ref0 = run_oracle(oracle, w, cells=[np.zeros(0)] * 4)
        check(out0, ref0, np.float32, "empty")
        full = ctx.step(*cells)
        check(full, run_oracle(oracle, w), np.float32, "full")
        half = tuple(c[: w.nc // 2] for c in cells)
        out = ctx.step(*half)
        check(out, run_oracle(oracle, w, cells=half), np.float32, "half")
        assert out["grad_x"].shape == (w.nc // 2,)
        with pytest.raises(ValueError):
            ctx.set_cells(*[np.zeros(w.nc + 1, np.float32)] * 4)


def test_cell_count_changes_across_block_shapes(oracle):
    """One context stepped with 0.3 M, then 1.4 M, then 0.9 M cells: each count
    cuts the cells into blocks of another size (2, 4, 3 cells per thread on a
    256-CU MI355X), so each one-pass step plans its regions from counts taken
    over a different block layout and overflows into the pool where they fall
    short.  Every step matches the oracle, and stepping the same cells again
    (regions now from a matching layout) is bitwise the same."""
    import dpep
    from dpep import workloads
    w = workloads.config3(seed=5, n_mov=1_400_000)
    cells = w.cells(np.float32)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh) as ctx:
        ctx.set_initial_density(w.d0n.astype(np.float32))
        for n in (300_000, 1_400_000, 900_000):
            sub = tuple(c[:n] for c in cells)
            out = ctx.step(*sub)
            again = ctx.step(*sub)
            for k in out:
                assert np.array_equal(out[k], again[k], equal_nan=True), f"{n}: {k}"
            check(out, run_oracle(oracle, w, cells=sub), np.float32, f"{n} cells")


def test_timings_and_kernel_times():
    import dpep
    from dpep import workloads
    w = workloads.small(3, seed=8, cells=50000, grid=256)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, step_timings=True) as ctx:
        ctx.set_cells(*w.cells(np.float32))
        ctx.set_profiling(4)
        for _ in range(4):
            ctx.compute()
        ctx.sync()
        kt = ctx.kernel_times_us()
        t = ctx.timings()
    assert set(kt) == set(dpep.KERNEL_KEYS)
    assert all(v > 0 for v in kt.values())
    assert kt["step"] >= kt["strip_acc"] + kt["col_pass"]
    assert set(t) == set(dpep.TIMING_KEYS) and t["total"] > 0
    # without DPEP_FLAG_STEP_TIMINGS (and without profiling) no step event is
    # recorded: the compute slot reads 0, the results are the same
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh) as ctx:
        out = ctx.step(*w.cells(np.float32))
        t0 = ctx.timings()
    assert t0["compute"] == 0.0 and np.isfinite(out["density"]).all()


def test_full_step_8192_columns(oracle):
    """float32 rows of 8192 bins: 2-row strips (the largest LDS tile, 128 KiB
    + 16 B), the 8192-point row DCT inside the accumulation, two gather rows
    at a time; cells of all sizes, some spanning more than a strip."""
    import dpep
    M, N = 64, 8192
    rng = np.random.default_rng(8192)
    nc = 40000
    xh, yh = 640.0, 81920.0
    sx = rng.uniform(0.5, 30.0, nc)
    sy = rng.uniform(2.0, 40.0, nc)
    px = rng.uniform(-5.0, xh, nc)
    py = rng.uniform(-5.0, yh, nc)
    cells = [a.astype(np.float32) for a in (px, py, sx, sy)]
    d0 = (0.3 * rng.random((M, N))).astype(np.float32)
    with dpep.Context(M, N, nc, 0.0, 0.0, xh, yh) as ctx:
        ctx.set_initial_density(d0)
        for k in range(2):       # twice: the side map must be left clean
            out = ctx.step(*cells)
    ref = oracle.step(*cells, M, N, 0.0, 0.0, xh, yh, d0n=d0)
    print(check(out, ref, np.float32, "64x8192"), flush=True)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_offset_die_with_oblong_bins(oracle, dtype):
    """A die whose lower-left corner is not the origin, bins 5 x 11.72 (the
    field weights carry bsx / bsy), 1024 x 256 bins (128 strips of 8 rows of
    256 columns), cells of all sizes including some past every die edge."""
    M, N = 1024, 256
    xl, yl = -1234.5, 777.25
    xh, yh = xl + 5.0 * M, yl + 3000.0
    rng = np.random.default_rng(1024 + 256)
    nc = 60000
    sx = rng.uniform(0.3, 25.0, nc)
    sy = rng.uniform(0.3, 60.0, nc)
    px = rng.uniform(xl - 10.0, xh, nc)
    py = rng.uniform(yl - 20.0, yh, nc)
    cells = [a.astype(dtype) for a in (px, py, sx, sy)]
    d0 = (0.4 * rng.random((M, N))).astype(dtype)

    class W:
        pass
    w = W()
    w.M, w.N, w.xl, w.yl, w.xh, w.yh, w.d0n = M, N, xl, yl, xh, yh, d0
    errs = check(run_gpu(w, dtype, cells=cells), run_oracle(oracle, w, dtype, cells=cells),
                 dtype, f"offset die {np.dtype(dtype).name}")
    print(errs, flush=True)


@pytest.mark.parametrize("stretch", [True, False])
def test_cells_at_the_lower_die_edges(oracle, stretch):
    """Small cells whose (stretched) corner lies below the die's lower x edge,
    its lower y edge, or both, by up to 1.3 bins, on a die whose corner is not
    the origin.  A float32 record keeps such a cell within a bin of the edge
    (offset + 1: one row early along x, a flag bit along y); one further out
    goes to the side map.  Two steps on one context (counted, then one pass)
    are bitwise equal, and both match the float64 oracle within tolerance."""
    M, N = 256, 512
    bsx, bsy = 4.0, 3.0
    xl, yl = 311.5, -97.25
    xh, yh = xl + bsx * M, yl + bsy * N
    rng = np.random.default_rng(77 + int(stretch))
    nc = 40000
    sx = rng.uniform(0.05, 1.3, nc) * bsx
    sy = rng.uniform(0.05, 1.3, nc) * bsy
    px = rng.uniform(xl, xh - 2 * bsx, nc)
    py = rng.uniform(yl, yh - 2 * bsy, nc)
    q = nc // 4
    # a quarter along the lower x edge, one along the lower y edge, one at
    # the corner; the rest anywhere
    px[:q] = xl + rng.uniform(-1.3, 0.5, q) * bsx
    py[q:2 * q] = yl + rng.uniform(-1.3, 0.5, q) * bsy
    px[2 * q:3 * q] = xl + rng.uniform(-1.3, 0.5, q) * bsx
    py[2 * q:3 * q] = yl + rng.uniform(-1.3, 0.5, q) * bsy
    cells = [a.astype(np.float32) for a in (px, py, sx, sy)]

    class W:
        pass
    w = W()
    w.M, w.N, w.xl, w.yl, w.xh, w.yh = M, N, xl, yl, xh, yh
    w.d0n = (0.3 * rng.random((M, N))).astype(np.float32)
    print(f"lower edges, stretch={stretch}", flush=True)
    errs = check(run_gpu(w, cells=cells, stretch=stretch),
                 run_oracle(oracle, w, cells=cells, stretch=stretch),
                 np.float32, f"lower edges stretch={stretch}")
    print(errs, flush=True)


def test_step_device_matches_host_step():
    """dpep_step_device on caller-owned device buffers (allocated through the
    same HIP runtime libdpep links) equals the host-buffer step; afterwards
    the context's own outputs are stale and dpep_get_outputs refuses them."""
    import dpep
    from conftest import DeviceBuffers
    from dpep import workloads
    lib = dpep.load_library()
    w = workloads.small(3, seed=9, cells=30000, grid=256)
    cells = w.cells(np.float32)
    ref = run_gpu(w)
    mn = w.M * w.N
    with DeviceBuffers() as db:
        dc = [db.upload(a) for a in cells]
        dfx, dfy, dden, dphi = (db.alloc(mn * 4) for _ in range(4))
        dgx, dgy = db.alloc(w.nc * 4), db.alloc(w.nc * 4)
        with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh) as ctx:
            ctx.set_initial_density(w.d0n.astype(np.float32))
            rc = lib.dpep_step_device(ctx.handle, *dc, w.nc, dfx, dfy, dden, dphi,
                                      dgx, dgy, None)
            assert rc == 0, dpep.last_error()
            ctx.sync()
            ctx._last_nc = w.nc
            with pytest.raises(RuntimeError, match="stale"):
                ctx.get_outputs()
        got = {}
        for name, p, n in (("field_x", dfx, mn), ("field_y", dfy, mn),
                           ("density", dden, mn), ("potential", dphi, mn),
                           ("grad_x", dgx, w.nc), ("grad_y", dgy, w.nc)):
            got[name] = db.download(p, n, np.float32).reshape(ref[name].shape)
    for k in got:
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-6, atol=1e-6 * np.abs(ref[k]).max())


def test_outputs_are_stale_after_new_cells():
    """Cells uploaded after a step make its outputs stale: dpep_get_outputs
    refuses them until the next compute; the forces returned are sized by
    the computed step's cell count."""
    import dpep
    from dpep import workloads
    w = workloads.small(3, seed=10, cells=5000, grid=64)
    px, py, sx, sy = w.cells(np.float32)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh) as ctx:
        ctx.set_cells(px, py, sx, sy)
        ctx.compute()
        full = ctx.get_outputs()
        assert full["grad_x"].shape == (w.nc,)
        ctx.set_cells(px[:100], py[:100], sx[:100], sy[:100])
        with pytest.raises(RuntimeError, match="stale"):
            ctx.get_outputs()
        ctx.compute()
        assert ctx.get_outputs()["grad_x"].shape == (100,)


@pytest.mark.parametrize("pinned", [False, True])
def test_positions_only_upload_keeps_the_sizes(pinned):
    """set_cells(px, py) (NULL sizes in dpep_set_cells) moves the cells and
    keeps the resident sizes: the step is bitwise the one of a full upload of
    the same cells, for fewer cells as well; sizes never sent, or sent for
    fewer cells, are refused (DPEP_ERR_STATE) and leave the context usable."""
    import dpep
    from dpep import workloads
    w = workloads.small(3, seed=13, cells=20000, grid=256)
    px, py, sx, sy = w.cells(np.float32)
    rng = np.random.default_rng(3)
    kw = dict(pinned=pinned)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, **kw) as ctx, \
            dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, **kw) as full:
        for c in (ctx, full):
            c.set_initial_density(w.d0n.astype(np.float32))
        with pytest.raises(RuntimeError, match="resident sizes"):
            ctx.set_cells(px, py)
        ctx.set_cells(px, py, sx, sy)
        for n in (w.nc, w.nc, 5000):
            qx = (px[:n] + rng.normal(0, 3, n)).astype(np.float32)
            qy = (py[:n] + rng.normal(0, 3, n)).astype(np.float32)
            a = ctx.step(qx, qy)
            b = full.step(qx, qy, sx[:n], sy[:n])
            for k in b:
                assert np.array_equal(a[k], b[k], equal_nan=True), f"{k} n={n}"
        ctx.set_cells(px[:100], py[:100], sx[:100], sy[:100])
        with pytest.raises(RuntimeError, match="resident sizes"):
            ctx.set_cells(px[:101], py[:101])
        a = ctx.step(px[:100], py[:100])
        b = full.step(px[:100], py[:100], sx[:100], sy[:100])
        assert all(np.array_equal(a[k], b[k]) for k in b)


@pytest.mark.parametrize("pinned", [False, True])
def test_pinned_context_and_scatter_density(oracle, pinned):
    """A pinned context (page-locked staging) gives the same outputs, and
    the scatter density (DPEP_FLAG_SCATTER_DENSITY) is the cells' density
    without the initial density."""
    import dpep
    from dpep import workloads
    w = workloads.small(3, seed=12, cells=20000, grid=256)
    px, py, sx, sy = w.cells(np.float32)
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, pinned=pinned,
                      scatter_density=True) as ctx:
        ctx.set_initial_density(w.d0n.astype(np.float32))
        if pinned:
            hc = ctx.host_cells()
            for k, a in zip(("px", "py", "sx", "sy"), (px, py, sx, sy)):
                hc[k][:w.nc] = a
            out = ctx.step(hc["px"][:w.nc], hc["py"][:w.nc], hc["sx"][:w.nc],
                           hc["sy"][:w.nc])
        else:
            out = ctx.step(px, py, sx, sy)
        raw = ctx.scatter_density()
    ref = run_oracle(oracle, w)
    check(out, ref, np.float32, f"pinned={pinned}")
    e = rel_linf(raw, oracle.density(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh))
    print(f"scatter density rel Linf {e:.3e}", flush=True)
    assert e <= 1e-5


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_c5_hundred_steps(oracle, dtype):
    import dpep
    from dpep import workloads
    w = workloads.config5()
    px, py = w.px.copy(), w.py.copy()
    sx, sy = w.sx.astype(dtype), w.sy.astype(dtype)
    ba = w.bsx * w.bsy
    worst = {}
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype) as ctx:
        ctx.set_initial_density(w.d0n.astype(dtype))
        for step in range(100):
            px, py = workloads.c5_displace(w, px, py, step)
            cells = (px.astype(dtype), py.astype(dtype), sx, sy)
            out = ctx.step(*cells)
            # size-independent invariant every step: all cells lie inside the
            # die, so the density carries exactly the cells' area
            mass = out["density"].astype(np.float64).sum() * ba
            area = float((sx.astype(np.float64) * sy).sum())
            assert mass == pytest.approx(area, rel=1e-5 if dtype == np.float32 else 1e-11)
            if step % 20 == 19 or step == 0:
                ref = oracle.step(*cells, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                                  d0n=w.d0n.astype(dtype))
                for k, v in check(out, ref, dtype, f"C5 step {step}").items():
                    worst[k] = max(worst.get(k, 0.0), v)
    print(f"C5 {np.dtype(dtype).name} 100 steps, worst of steps 0,19,..,99: " +
          " ".join(f"{k}={v:.2e}" for k, v in worst.items()))


# --------------------------------------------------------------------------
# fixed-cell initial density D0 on the GPU
# --------------------------------------------------------------------------
def _fixed_oracle(oracle, w, fx, fy, fw, fh, target):
    """D0n = target * exact overlap / bin area: the oracle's density of the
    fixed cells with no stretch and ratio 1."""
    return target * oracle.density(np.asarray(fx, np.float64), np.asarray(fy, np.float64),
                                   np.asarray(fw, np.float64), np.asarray(fh, np.float64),
                                   w.M, w.N, w.xl, w.yl, w.xh, w.yh, stretch=False)


@pytest.mark.parametrize("cfg,grid,dtype", [(1, 512, np.float32), (3, 2048, np.float32),
                                            (1, 256, np.float64)])
def test_fixed_cells_density(oracle, cfg, grid, dtype):
    import dpep
    from dpep import workloads
    w = workloads.small(cfg, seed=9, cells=1000, grid=grid)
    mx, my, mw, mh = (np.asarray(a, dtype) for a in w.meta["fixed_cells"])
    # plus edge cases: outside the die, straddling its border, zero size,
    # exactly on bin edges, a copy of an existing macro (overlap)
    bs = w.bsx
    ex = np.array([-500.0, w.xh - 10 * bs, 3 * bs, 5 * bs, mx[0]], dtype)
    ey = np.array([-500.0, 4 * bs, 7 * bs, 9 * bs, my[0]], dtype)
    ew = np.array([100.0, 40 * bs, 0.0, 2 * bs, mw[0]], dtype)
    eh = np.array([100.0, 3 * bs, 5.0, 3 * bs, mh[0]], dtype)
    fx, fy = np.concatenate([mx, ex]), np.concatenate([my, ey])
    fw, fh = np.concatenate([mw, ew]), np.concatenate([mh, eh])
    target = 0.9
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype) as ctx:
        ctx.set_fixed_cells(fx, fy, fw, fh, target)
        out = ctx.step(*w.cells(dtype))
        ctx.set_fixed_cells(fx, fy, fw, fh, target)      # B left clean: same again
        out2 = ctx.step(*w.cells(dtype))
    d0 = _fixed_oracle(oracle, w, fx, fy, fw, fh, target)
    px, py, sx, sy = w.cells(dtype)
    ref = oracle.step(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                      d0n=d0.astype(dtype))
    check(out, ref, dtype, f"fixed C{cfg}")
    assert np.array_equal(out["density"], out2["density"])
    # no movable cells: the density is D0 itself
    with dpep.Context(w.M, w.N, 1, w.xl, w.yl, w.xh, w.yh, dtype=dtype) as ctx:
        ctx.set_fixed_cells(fx, fy, fw, fh, target)
        only = ctx.step(*(np.zeros(0, dtype),) * 4)
    assert rel_linf(only["density"], d0) <= TOL[dtype][0]


def test_fixed_cells_empty_and_errors():
    import dpep
    with dpep.Context(16, 16, 10, 0.0, 0.0, 160.0, 160.0) as ctx:
        ctx.set_initial_density(np.ones((16, 16), np.float32))
        ctx.set_fixed_cells(*(np.zeros(0, np.float32),) * 4)   # no fixed cells
        out = ctx.step(*(np.zeros(0, np.float32),) * 4)
        assert not out["density"].any()
        with pytest.raises(ValueError):
            ctx.set_fixed_cells(*(np.zeros(1, np.float32),) * 4, target_density=-1.0)
