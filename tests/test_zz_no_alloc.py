"""GPU: dpep_step_device_noalloc (the entry point that allocates nothing,
its scratch in one device array of the library) against dpep_step_device on
the same device buffers: two calls in a row, the second with fewer cells,
float32 and float64; every output must match bit for bit: both run the
same kernels on the same inputs, with the same device-built tables, and
integer accumulation makes the density independent of the order records
are placed in.  Also: a problem too large for the array
is refused with its size, and a NULL initial density means zero."""
import numpy as np
import pytest

from conftest import DeviceBuffers, rel_l2, rel_linf

pytestmark = pytest.mark.gpu

OUTS = ("field_x", "field_y", "density", "potential", "grad_x", "grad_y")


def _noalloc(lib, w, dtype, nc_max, d0, cells, nc, outs, flags=0):
    dt = 0 if dtype == np.float32 else 1
    return lib.dpep_step_device_noalloc(w.M, w.N, w.xl, w.yl, w.xh, w.yh, dt, flags, nc_max,
                                        d0, *cells, nc, *(outs[k] for k in OUTS), None)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_noalloc_matches_step_device(oracle, dtype):
    import dpep
    from dpep import workloads
    lib = dpep.load_library()
    w = workloads.small(3, seed=31, cells=60000, grid=512)
    n1, n2 = w.nc, w.nc // 3
    esz = np.dtype(dtype).itemsize
    mn = w.M * w.N
    print(f"noalloc dtype={np.dtype(dtype).name} grid={w.M} cells={n1},{n2}", flush=True)
    with DeviceBuffers() as db:
        px, py, sx, sy = w.cells(dtype)
        d0 = db.upload(w.d0n.astype(dtype))

        def outs():
            return {k: db.alloc((w.nc if k.startswith("grad") else mn) * esz) for k in OUTS}

        def fetch(o, nc):
            return {k: db.download(o[k], nc if k.startswith("grad") else mn, dtype)
                    for k in OUTS}

        with dpep.Context(w.M, w.N, n1, w.xl, w.yl, w.xh, w.yh, dtype=dtype) as ctx:
            ctx.set_initial_density(w.d0n.astype(dtype))
            for call, nc in enumerate((n1, n2)):
                shift = dtype(0.37 * call)          # the cells move between calls
                cells = [db.upload(a[:nc] + (shift if i < 2 else 0))
                         for i, a in enumerate((px, py, sx, sy))]
                oa, ob = outs(), outs()
                rc = lib.dpep_step_device(ctx.handle, *cells, nc,
                                          *(oa[k] for k in OUTS), None)
                assert rc == 0, dpep.last_error()
                ctx.sync()
                rc = _noalloc(lib, w, dtype, n1, d0, cells, nc, ob)
                assert rc == 0, dpep.last_error()
                db.sync()
                a, b = fetch(oa, nc), fetch(ob, nc)
                for k in OUTS:
                    d = float(np.abs(b[k].astype(np.float64) - a[k]).max()) if nc else 0.0
                    print(f"call {call} nc={nc} {k}: max |noalloc - step_device| {d:.3e}",
                          flush=True)
                    assert np.array_equal(a[k], b[k]), (call, k, d)
                if call == 1:
                    c = [np.asarray(v[:nc]) + (shift if i < 2 else 0)
                         for i, v in enumerate((px, py, sx, sy))]
                    ref = oracle.step(*c, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                                      d0n=w.d0n.astype(dtype))
                    tl, tf = (1e-5, 1e-4) if dtype == np.float32 else (1e-10, 1e-9)
                    assert rel_linf(b["density"].reshape(w.M, w.N), ref["density"]) <= tl
                    assert rel_l2(b["grad_x"], ref["grad_x"]) <= tf


def test_noalloc_limits_and_zero_initial_density(oracle):
    import dpep
    from dpep import workloads
    lib = dpep.load_library()
    w = workloads.small(3, seed=32, cells=20000, grid=256)
    mn = w.M * w.N
    with DeviceBuffers() as db:
        cells = [db.upload(a) for a in w.cells(np.float32)]
        o = {k: db.alloc((w.nc if k.startswith("grad") else mn) * 4) for k in OUTS}
        # NULL initial density = zero
        assert _noalloc(lib, w, np.float32, w.nc, None, cells, w.nc, o) == 0, \
            dpep.last_error()
        db.sync()
        dens = db.download(o["density"], mn, np.float32).reshape(w.M, w.N)
        ref = oracle.density(*w.cells(np.float32), w.M, w.N, w.xl, w.yl, w.xh, w.yh)
        assert rel_linf(dens, ref) <= 1e-5
        # 4096 x 4096 float32 needs more than the array holds: refused, nothing run
        class Big:
            M = N = 4096
            xl, yl, xh, yh = w.xl, w.yl, w.xh, w.yh
        rc = _noalloc(lib, Big, np.float32, w.nc, None, cells, w.nc, o)
        assert rc == 1 and "MiB" in dpep.last_error()
        # every output the step computes must be given
        o2 = dict(o, grad_x=None)
        assert _noalloc(lib, w, np.float32, w.nc, None, cells, w.nc, o2) == 1
        # ... unless the flags drop it (NO_GATHER = 8)
        assert _noalloc(lib, w, np.float32, w.nc, None, cells, w.nc, o2, flags=8) == 0
        db.sync()
