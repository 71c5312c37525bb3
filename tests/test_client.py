"""Shared-memory client (dpep.scatter_ttnn_client) on the CPU, against the
oracle-backed loopback server: wire layout, the per-step protocol, timing
dicts, error paths (integration/scatter_ttnn_client.py:293-531 of the
reference), the DREAMPlace adapter's cell selection (:611-640), and the real
server binary's start-up failure without a GPU."""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

from conftest import PKG, ROOT, rel_l2, rel_linf

from dpep import shm as S
from dpep import workloads
from dpep.scatter_ttnn_client import ScatterTTNNClient

LOOPBACK = [sys.executable, os.path.join(ROOT, "tests", "loopback_server.py")]
SERVER_BIN = os.path.join(PKG, "dpep", "density_scatter_hip_server")


def _w(seed, cells, grid):
    return workloads.small(3, seed=seed, cells=cells, grid=grid)


def _client(tmp_path, w, nc_max=None, **kw):
    return ScatterTTNNClient(ipc_dir=str(tmp_path / "ipc"), num_bins_x=w.M,
                             num_bins_y=w.N, nc_max=nc_max or w.nc, xl=w.xl,
                             yl=w.yl, xh=w.xh, yh=w.yh, server_binary=LOOPBACK,
                             as_torch=False, ready_timeout=120, **kw)


def test_layout_v1_matches_reference_formula():
    # header 64 B, four position slots of ceil(nc/1024)*1024 floats, then
    # field_x, field_y, init_density of M*N floats (reference client :224-271)
    lay = S.Layout(16, 32, 1500, version=1)
    assert lay.soa == 2048
    assert lay.offset("px") == 64
    assert lay.offset("sy") == 64 + 3 * 2048 * 4
    assert lay.offset("field_x") == 64 + 4 * 2048 * 4
    assert lay.offset("init_density") == 64 + 4 * 2048 * 4 + 2 * 16 * 32 * 4
    assert lay.total_size == 64 + 4 * 2048 * 4 + 3 * 16 * 32 * 4
    with pytest.raises(KeyError):
        lay.offset("density")
    v2 = S.Layout(16, 32, 1500, version=2)
    assert v2.offset("density") == lay.total_size
    assert v2.offset("grad_y") == lay.total_size + 2 * 16 * 32 * 4 + 2048 * 4
    assert v2.total_size == lay.total_size + 2 * 16 * 32 * 4 + 2 * 2048 * 4
    assert struct.calcsize(S.HDR_TIMING_FMT) == 48


def test_loopback_steps_match_oracle(tmp_path, oracle):
    w = _w(3, 900, 32)
    c = _client(tmp_path, w, nc_max=max(1000, w.nc))
    c.set_initial_density(w.d0n)
    c.start()
    try:
        args = open(tmp_path / "ipc" / "args.txt").read().split()
        assert args[:3] == ["32", "32", str(max(1000, w.nc))] and float(args[6]) == w.xh
        for k in range(2):
            px, py, sx, sy = w.cells(np.float32)
            px = px + np.float32(k)            # move cells between steps
            fx, fy, timing = c.call(px, py, sx, sy)
            ref = oracle.step(px.astype(np.float64), py, sx, sy, w.M, w.N, w.xl, w.yl,
                              w.xh, w.yh, d0n=w.d0n)
            assert rel_l2(fx, ref["field_x"]) < 1e-6
            assert rel_l2(fy, ref["field_y"]) < 1e-6
            assert timing["gather_mode"] == "hip"
            for key in ("pos_write_ms", "kernel_wait_ms", "field_read_ms",
                        "total_server_ms", "total_client_ms", "ttnn_compute_ms"):
                assert key in timing
        full = c.call_full(px, py, sx, sy)
        assert rel_linf(full["density"], ref["density"]) < 1e-6
        assert rel_linf(full["potential"], ref["potential"]) < 1e-6
        assert full["grad_x"].shape == (w.nc,)
        assert rel_l2(full["grad_x"], ref["grad_x"]) < 1e-6
        summ = c.timing_summary(n_warmup=1)
        assert summ["n_iters"] == 3 and summ["n_timed"] == 2
        assert summ["gather_mode"] == "hip" and "total_client_ms_mean" in summ
    finally:
        proc = c._proc
        c.stop()
    assert proc.wait(timeout=30) == 0
    assert not os.path.exists(c.shm_path)


def test_fewer_cells_than_capacity(tmp_path, oracle):
    w = _w(4, 600, 16)
    c = _client(tmp_path, w, nc_max=2000)
    c.start()
    try:
        px, py, sx, sy = w.cells(np.float32)
        out = c.call_full(px, py, sx, sy)
        ref = oracle.step(px, py, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh)
        assert rel_linf(out["density"], ref["density"]) < 1e-6
        assert out["grad_y"].shape == (w.nc,) and w.nc <= 2000
        with pytest.raises(ValueError):
            c.call(*(np.zeros(2001, np.float32),) * 4)
    finally:
        c.stop()


def test_stale_ready_flag_is_removed(tmp_path):
    w = _w(5, 100, 8)
    ipc = tmp_path / "ipc"
    ipc.mkdir()
    (ipc / "ready.flag").write_text("STALE\n")
    c = _client(tmp_path, w)
    c.start()
    try:
        assert (ipc / "ready.flag").read_text() == "READY\n"
    finally:
        c.stop()


def test_error_paths(tmp_path, monkeypatch):
    w = _w(6, 100, 8)
    with pytest.raises(FileNotFoundError):
        ScatterTTNNClient(ipc_dir=str(tmp_path / "a"), num_bins_x=8, num_bins_y=8,
                          nc_max=10, server_binary=str(tmp_path / "none")).start()
    with pytest.raises(ValueError):
        ScatterTTNNClient(ipc_dir=str(tmp_path / "b"), num_bins_x=8,
                          num_bins_y=8).start()
    with pytest.raises(RuntimeError):
        _client(tmp_path, w).call(*(np.zeros(4, np.float32),) * 4)

    monkeypatch.setenv("LOOPBACK_MODE", "exit")
    with pytest.raises(RuntimeError, match="code 3"):
        _client(tmp_path, w).start()

    monkeypatch.setenv("LOOPBACK_MODE", "noready")
    c = _client(tmp_path, w)
    c.ready_timeout = 1.0
    with pytest.raises(TimeoutError):
        c.start()
    assert c._proc.poll() is not None            # killed, not left behind

    monkeypatch.setenv("LOOPBACK_MODE", "hang")
    c = _client(tmp_path, w, step_timeout=0.5)
    c.start()
    try:
        with pytest.raises(TimeoutError):
            c.call(*w.cells(np.float32))
    finally:
        proc = c._proc
        c.stop()
    assert proc.wait(timeout=30) == 0            # QUIT still ends a stuck server


def test_returns_torch_when_asked(tmp_path):
    torch = pytest.importorskip("torch")
    w = _w(7, 50, 8)
    c = _client(tmp_path, w)
    c.as_torch = True
    c.start()
    try:
        fx, fy, _ = c.call(*w.cells(np.float32))
        assert isinstance(fx, torch.Tensor) and fx.shape == (8, 8)
    finally:
        c.stop()


def test_dreamplace_adapter_selects_movable_and_filler(tmp_path, oracle):
    """The patched forward passes [movable | filler] cells with their
    original sizes (clamped + 2*offset) and the die, grid and initial density
    taken from the call (reference :611-640, :786-795)."""
    torch = pytest.importorskip("torch")
    from dpep import scatter_ttnn_client as stc

    rng = np.random.default_rng(11)
    n_mov, n_fix, n_fil = 40, 5, 15
    n = n_mov + n_fix + n_fil
    M = N = 16
    die = 160.0
    pos = torch.from_numpy(np.concatenate([rng.uniform(0, 150, n), rng.uniform(0, 150, n)]))
    sx = rng.uniform(1, 20, n)
    sy = rng.uniform(1, 20, n)
    # DREAMPlace clamps to sqrt2*bin and keeps offset = (size - clamped)/2
    bs = die / M
    csx, csy = np.maximum(sx, np.sqrt(2) * bs), np.maximum(sy, np.sqrt(2) * bs)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    init = rng.uniform(0, 5, (M, N))

    class Ctx:
        pass

    client = _client(tmp_path, _w(0, n, M), nc_max=n)
    client.M = client.N = 0                       # taken from the call
    fwd = stc.make_forward(client).__func__
    try:
        fwd(Ctx(), pos, t(csx), t(csy), t((sx - csx) / 2), t((sy - csy) / 2), None,
            None, None, t(init), 1.0, 0.0, 0.0, die, die, bs, bs, n_mov, n_fil,
            0, None, M, N, 0, 0, 0, 0, False, None)
        sel = np.r_[0:n_mov, n - n_fil:n]
        p = pos.numpy()
        ref = oracle.step(p[:n][sel], p[n:][sel], sx[sel], sy[sel], M, N, 0.0, 0.0,
                          die, die, d0n=init / (bs * bs))
        out = client.last_outputs
        assert rel_linf(out["density"], ref["density"]) < 1e-5
        assert rel_l2(out["field_x"], ref["field_x"]) < 1e-5
    finally:
        client.stop()


def test_patch_dreamplace_needs_dreamplace(tmp_path):
    from dpep import scatter_ttnn_client as stc
    try:
        import dreamplace  # noqa: F401
        pytest.skip("DREAMPlace is installed")
    except ImportError:
        pass
    with pytest.raises(ImportError):
        stc.patch_dreamplace(ipc_dir=str(tmp_path / "ipc"), num_cells=10)
    assert stc.get_timing_summary() == {}
    stc.teardown()


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible: start-up would succeed")
def test_real_server_fails_loudly_without_gpu(tmp_path):
    if not os.path.exists(SERVER_BIN):
        pytest.skip("server binary not built")
    r = subprocess.run([SERVER_BIN], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "Usage" in r.stderr
    w = _w(8, 10, 8)
    c = _client(tmp_path, w)
    c.server_binary = SERVER_BIN
    with pytest.raises(RuntimeError, match="code 1"):
        c.start()
