"""GPU: the drop-in boundary end to end -- density_scatter_hip_server driven
by ScatterTTNNClient over the shared-memory protocol, and the client's
in-process mode over the C ABI -- against the float64 oracle on the same
seeded cells (float32 tolerances: density/potential rel L-inf <= 1e-5,
fields/forces rel L2 <= 1e-4)."""
import os

import numpy as np
import pytest

from conftest import PKG, rel_l2, rel_linf

from dpep import workloads
from dpep.scatter_ttnn_client import ScatterTTNNClient

pytestmark = pytest.mark.gpu

SERVER_BIN = os.path.join(PKG, "dpep", "density_scatter_hip_server")


def _check(out, ref):
    for k in ("density", "potential"):
        e = rel_linf(out[k], ref[k])
        assert e <= 1e-5, f"{k} rel Linf {e:.3e}"
    for k in ("field_x", "field_y", "grad_x", "grad_y"):
        e = rel_l2(out[k], ref[k])
        assert e <= 1e-4, f"{k} rel L2 {e:.3e}"


@pytest.mark.parametrize("inprocess", [False, True])
def test_client_against_oracle(tmp_path, oracle, inprocess):
    if not inprocess and not os.path.exists(SERVER_BIN):
        pytest.fail(f"server binary missing: {SERVER_BIN}")
    w = workloads.small(3, seed=21, cells=30000, grid=256)
    print(f"client inprocess={inprocess} cells={w.nc} grid={w.M}", flush=True)
    c = ScatterTTNNClient(ipc_dir=str(tmp_path / "ipc"), num_bins_x=w.M,
                          num_bins_y=w.N, nc_max=w.nc + 5000, xl=w.xl, yl=w.yl,
                          xh=w.xh, yh=w.yh, inprocess=inprocess,
                          server_binary=SERVER_BIN, as_torch=False,
                          ready_timeout=120, step_timeout=60)
    c.set_initial_density(w.d0n)
    c.start()
    try:
        px, py, sx, sy = w.cells(np.float32)
        rng = np.random.default_rng(5)
        for k in range(3):
            # cells move between steps, as in a placement run
            pxk = (px + rng.normal(0, 2, px.size)).astype(np.float32)
            out = c.call_full(pxk, py, sx, sy)
            ref = oracle.step(pxk, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                              d0n=w.d0n.astype(np.float32))
            _check(out, ref)
        # positions alone: the sizes stay those of the last call that sent
        # them (the shm or staging size slots are scribbled over to show they
        # are not re-read)
        if inprocess:
            staged = c._ctx.host_cells()
            staged["sx"][:] = -7.0
            staged["sy"][:] = np.nan
        else:
            c._views["sx"][:] = -7.0
            c._views["sy"][:] = np.nan
        for k in range(2):
            pxk = (px + rng.normal(0, 2, px.size)).astype(np.float32)
            out = c.call_full(pxk, py)
            ref = oracle.step(pxk, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                              d0n=w.d0n.astype(np.float32))
            _check(out, ref)
        # fewer cells than before: the tail of the previous step is gone
        n2 = w.nc // 3
        out = c.call_full(px[:n2], py[:n2], sx[:n2], sy[:n2])
        ref = oracle.step(px[:n2], py[:n2], sx[:n2], sy[:n2], w.M, w.N, w.xl, w.yl,
                          w.xh, w.yh, d0n=w.d0n.astype(np.float32))
        _check(out, ref)
        t = c.timing_summary(n_warmup=1)
        assert t["gather_mode"] == "hip" and t["n_iters"] == 6
    finally:
        c.stop()


def test_server_dumps_replay_to_the_same_density(tmp_path, monkeypatch, oracle):
    """EXPORT_POS_PATH / EXPORT_DENSITY_PATH from the server, replayed through
    dpep.replay: the same cells (bitwise) and the same density (the step is
    deterministic).  The density dump is the cells' density before the
    initial density is added, as the reference's (server :1676-1695)."""
    from dpep import replay
    if not os.path.exists(SERVER_BIN):
        pytest.fail(f"server binary missing: {SERVER_BIN}")
    pos = tmp_path / "pos.bin"
    dens = tmp_path / "dens.bin"
    monkeypatch.setenv("EXPORT_POS_PATH", str(pos))
    monkeypatch.setenv("EXPORT_DENSITY_PATH", str(dens))
    w = workloads.small(3, seed=23, cells=20000, grid=256)
    c = ScatterTTNNClient(ipc_dir=str(tmp_path / "ipc"), num_bins_x=w.M,
                          num_bins_y=w.N, nc_max=w.nc, xl=w.xl, yl=w.yl,
                          xh=w.xh, yh=w.yh, server_binary=SERVER_BIN, as_torch=False,
                          ready_timeout=120, step_timeout=60)
    c.set_initial_density(w.d0n)
    c.start()
    try:
        px, py, sx, sy = w.cells(np.float32)
        out = c.call_full(px, py, sx, sy)
    finally:
        c.stop()
    d = replay.read_positions(str(pos) + ".iter1.bin")
    assert d.nc == w.nc and np.array_equal(d.px, px) and np.array_equal(d.sy, sy)
    dumped = replay.read_density(str(dens), w.M, w.N)
    raw = oracle.density(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh)
    e = rel_linf(dumped, raw)
    print(f"dump vs oracle density without D0: rel Linf {e:.3e}", flush=True)
    assert e <= 1e-5
    r = replay.replay(d, w.d0n.astype(np.float32))
    assert np.array_equal(r["scatter_density"], dumped)
    assert np.array_equal(r["density"], out["density"])
    assert np.array_equal(r["field_x"], out["field_x"])


@pytest.mark.parametrize("inprocess", [False, True])
def test_cpu_dct_mode_sends_the_density_without_d0(tmp_path, monkeypatch, oracle,
                                                   inprocess):
    """CPU_DCT=1 (reference server :1757-1788): the field_x slot carries the
    cells' density without the initial density, field_y is zero; the v2
    density slot keeps rho + D0."""
    monkeypatch.setenv("CPU_DCT", "1")
    w = workloads.small(3, seed=25, cells=30000, grid=256)
    print(f"cpu_dct inprocess={inprocess} cells={w.nc} grid={w.M}", flush=True)
    c = ScatterTTNNClient(ipc_dir=str(tmp_path / "ipc"), num_bins_x=w.M,
                          num_bins_y=w.N, nc_max=w.nc, xl=w.xl, yl=w.yl,
                          xh=w.xh, yh=w.yh, inprocess=inprocess,
                          server_binary=SERVER_BIN, as_torch=False,
                          ready_timeout=120, step_timeout=60)
    c.set_initial_density(w.d0n)
    c.start()
    try:
        px, py, sx, sy = w.cells(np.float32)
        for k in range(2):
            pxk = px + np.float32(3 * k)
            fx, fy, _ = c.call(pxk, py, sx, sy)
            raw = oracle.density(pxk, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh)
            e = rel_linf(fx, raw)
            print(f"step {k}: field_x slot vs density without D0 rel Linf {e:.3e}",
                  flush=True)
            assert e <= 1e-5
            assert not np.asarray(fy).any()
            dens = c.last_outputs["density"]
            ref = oracle.density(pxk, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh,
                                 d0n=w.d0n.astype(np.float32))
            assert rel_linf(dens, ref) <= 1e-5
    finally:
        c.stop()


def test_dreamplace_adapter_forces_on_gpu(tmp_path):
    """The patched forward and backward (dpep.scatter_ttnn_client) through
    the shm server on the 1.1M-cell 2048^2 workload: the gradient the
    backward returns equals -grad_pos times the oracle's per-cell gather
    (rel L2 <= 1e-4), terminals get zero.  Runs in a child process because
    the adapter imports torch, whose bundled HIP runtime must not share a
    process with libdpep's."""
    import json
    import subprocess
    import sys
    if not os.path.exists(SERVER_BIN):
        pytest.fail(f"server binary missing: {SERVER_BIN}")
    script = os.path.join(os.path.dirname(__file__), "adapter_gpu_run.py")
    r = subprocess.run([sys.executable, "-u", script, str(tmp_path / "ipc")],
                       capture_output=True, text=True, timeout=900)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0
    res = json.loads(r.stdout.strip().splitlines()[-1])
    for sfx in ("", "_moved"):           # sizes sent, then positions alone
        assert res["grad_x" + sfx] <= 1e-4 and res["grad_y" + sfx] <= 1e-4
        assert res["field_x" + sfx] <= 1e-4 and res["field_y" + sfx] <= 1e-4
        assert res["terminals_zero" + sfx]
    assert not res["sizes_kept"] and res["sizes_kept_moved"]
